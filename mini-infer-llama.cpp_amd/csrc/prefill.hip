// prefill.hip -- fused causal ATTN_QK -> SOFTMAX -> ATTN_KQV for n_tokens > 1
// queries (src/ops_cpu.cpp:304-410) on the matrix cores of gfx950: float
// products on v_mfma_f32_32x32x2f32 (the default), or an opt-in form whose
// float operands are split into bf16 pairs for v_mfma_f32_32x32x16_bf16.
//
// Work decomposition. A query block is 32 consecutive queries of one head; it
// sees ceil((n_past + 32 (i + 1)) / 32) key tiles of 32 keys (causal). One
// workgroup owns the query blocks i and NQ - 1 - i of one head, so every
// workgroup has the same number of tiles (NQ + 1 + 2 n_past / 32 when the
// blocks are full). Its NW waves work through that list of (block, tile)
// units: wave w starts with unit w and then takes units in order from an LDS
// counter, so a wave that is served faster takes more (or, in deterministic
// launches, units w + NW, w + 2 NW, ...); a wave's units cross from block i to
// block NQ - 1 - i at most once, where it parks its first block's partial
// result in LDS.
//
// Per unit (lane = (c = lane % 32, kh = lane / 32)):
//   1. the key tile's 32 K rows come into the wave's LDS tile by buffer_load
//      ... lds (no registers), four rows per instruction, 16-byte slots XOR-
//      swizzled by row; lane (c, kh) then reads K[key c][kh D/2 ..] from it,
//      conflict-free, as the A operand. V goes straight to registers in the
//      A layout of the PV product: lane (c, kh) holds V[key][NDB c + db] for
//      the 16 keys 8(t/4) + 4kh + t%4, one load of NDB = D/32 consecutive
//      elements per key (so row c of output block db is dim NDB c + db);
//   2. S^T = K . Q^T with D/2 v_mfma_f32_32x32x2f32: B = the block's queries,
//      pre-scaled by scale*log2(e) (staged once per workgroup in LDS at
//      head_dim 64);
//   3. causal mask (key > n_past + query; only on tiles that reach past a
//      query of the block) and online softmax in base 2: a lane holds 16 keys
//      of query c and its partner lane (lane ^ 32) the other 16 (one
//      permlane32 swap combines them); O is rescaled only when some row's
//      maximum moved;
//   4. O^T += V^T . P^T with 16 MFMAs per 32 output dims; S^T leaves step 3 in
//      the B-operand layout of this product (register r of a lane = key
//      8(r/4) + 4kh + r%4), so P needs no shuffle.
// The units are software-pipelined: while unit u's softmax runs on the vector
// ALUs, the next unit's QK products run on the matrix cores (the two are
// interleaved instruction by instruction: the products form one dependent
// chain, which would otherwise hold the wave's issue until it drains); the K
// tile after that is requested as soon as the LDS tile has been read, V after
// the PV products that consumed the previous one.
// At the end the waves' (m, l, O) records meet in LDS and each block's output
// is merged with the stable rescaling; nothing else leaves the workgroup. Two
// waves per SIMD at head_dim 64 (one at 128) let one wave's vector work run
// under the other's matrix-core work.
#include <type_traits>

#include "attn_common.h"
#include "kernels.h"

namespace mi {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;
typedef __attribute__((address_space(3))) f16x8 lds_f16x8;
typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) unsigned lds_u32;

namespace {

// 16 bytes per lane from r at vo (per lane, range-checked) + so (wave-uniform)
// into LDS at lds + 16 * lane. (A plain function: in the kernel template the
// host pass rejects the builtin's LDS pointer and drops the kernel silently.)
__device__ inline void dma16(rsrc_t r, lds_t* lds, unsigned vo, unsigned so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, vo, so, 0, 0);
}

// x and lane ^ 32's x, in some order, in one v_permlane32_swap (no LDS round
// trip): swapping the upper half of one copy of x with the lower half of
// another leaves each lane holding both. Written as asm: the compiler's
// builtin for this instruction drops one of its two results when they are
// used as floats. The s_nop gives the two wait states a VALU write of an
// operand needs before the swap reads it.
__device__ inline void xor32_pair(float x, float& a, float& b) {
  float y = x;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  a = x;
  b = y;
}
__device__ inline float xor32_max(float x) {
  float a, b;
  xor32_pair(x, a, b);
  return fmaxf(a, b);
}
__device__ inline float xor32_sum(float x) {
  float a, b;
  xor32_pair(x, a, b);
  return a + b;
}

// Eight floats as hi + lo bf16 pairs: hi = bf16(x) rounded to nearest even,
// lo = bf16(x - hi) (x - hi is exact in float), so |x - hi - lo| <= 2^-17 |x|.
__device__ inline void split8(const float* x, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const __bf16 h = (__bf16)x[i];
    hi[i] = h;
    lo[i] = (__bf16)(x[i] - (float)h);
  }
}

// F16 cache values (exact in f16) as f16, and float values x as an f16 pair
// hi = RNE(x), lo = RNE(x - hi) (|x - hi - lo| <= 2^-22 |x| while lo is
// normal, 2^-25 absolute below).
__device__ inline void pack8h(const float* x, f16x8& v) {
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (_Float16)x[i];
}
__device__ inline void split8h(const float* x, f16x8& hi, f16x8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 h = (_Float16)x[i];
    hi[i] = h;
    lo[i] = (_Float16)(x[i] - (float)h);
  }
}
// acc += a . b over 16 k-values, a exact in f16 (the F16 cache operand), b
// a float operand split into an f16 pair: a.b_lo + a.b_hi, two
// v_mfma_f32_32x32x16_f16 (f16 products are exact in the float accumulator).
__device__ inline floatx16 mfma2h(const f16x8& a, const f16x8& bh, const f16x8& bl, floatx16 acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bh, acc, 0, 0, 0);
}

// acc += a . b over 16 k-values with float inputs split into bf16 pairs:
// a_lo.b_hi + a_hi.b_lo + a_hi.b_hi (the a_lo.b_lo term, below 2^-18 of the
// product, is dropped), three v_mfma_f32_32x32x16_bf16 in that order.
__device__ inline floatx16 mfma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, const bf16x8& bl,
                                 floatx16 acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
}

}  // namespace

template <int D, typename KT, int NW>
struct PrefillCfg {
  static constexpr int ELT = (int)sizeof(KT);
  static constexpr int HALF = D / 2;                   // QK MFMA steps
  static constexpr int NDB = D / 32;                   // PV output blocks of 32 dims
  static constexpr int NV = 16 * NDB;                  // V values per lane per tile
  static constexpr int NVL = 16;                       // V loads per lane per tile (one per key)
  static constexpr int RB = D * ELT;                   // bytes per K row
  static constexpr int NSLOT = RB / 16;                // 16-byte slots per K row
  static constexpr int KTILE = kPrefillKeys * RB;      // bytes of one K tile
  static constexpr int NDK = KTILE / 1024;             // 1 KB loads per K tile
  static constexpr int HSL = HALF * ELT / 16;          // slots per half row
  static constexpr int RS = D + 4;                     // record row stride (floats)
  static constexpr int RECF = kPrefillRows * RS + 2 * kPrefillRows;  // O rows, m, l
  static constexpr int RECB = RECF * 4;
  static constexpr int REG = (KTILE > RECB ? KTILE : RECB);  // K tile, later block-qz record
  static constexpr bool QLDS = D == 64;                // queries staged in LDS
  static constexpr int QRS = D + 4;                    // staged query row stride (floats)
  // LDS layout (bytes): block-qa records, per-wave K tile / block-qz record,
  // staged queries, unit counter
  static constexpr int L_REC0 = 0;
  static constexpr int L_REG = L_REC0 + NW * RECB;
  static constexpr int L_Q = L_REG + NW * REG;
  static constexpr int L_CTR = L_Q + (QLDS ? 2 * kPrefillRows * QRS * 4 : 0);
  static constexpr int LDS = L_CTR + 16;
  // vector memory operations a wave issues after a K tile request and before
  // the next tile's wait (the V loads of one unit)
  static constexpr int WAIT_K = NVL;
  static_assert(KTILE % 1024 == 0, "1 KB load granularity");
  static_assert(REG % 16 == 0 && RECB % 16 == 0, "16-byte alignment");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int D, typename KT, int NW, bool SPLIT>
__global__ __launch_bounds__(NW* kWave) void prefill_kernel(const PrefillParams p) {
  typedef PrefillCfg<D, KT, NW> C;
  constexpr int HALF = C::HALF, NDB = C::NDB, NV = C::NV, RS = C::RS, ELT = C::ELT;
  constexpr int NSLOT = C::NSLOT;

  extern __shared__ __attribute__((aligned(16))) char lds_raw[];
  lds_t* const lds = (lds_t*)lds_raw;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int col = lane & 31;
  const int kh = lane >> 5;

  // workgroup -> (head h, query blocks qa and qz): pairs (j, NQ - 1 - j), or
  // with p.lone the last block alone and then pairs (j, NQ - 2 - j). A lone
  // middle block has qz == qa.
  const int h = blockIdx.x % p.n_head;
  const int j = blockIdx.x / p.n_head;
  const bool last_alone = p.lone && j == 0;
  const int qa = last_alone ? p.n_qblocks - 1 : j - p.lone;
  const int qz = last_alone ? qa : p.n_qblocks - 1 - p.lone - qa;
  const int n_kv = p.n_past + p.n_tokens;
  auto tiles = [&](int i) {
    return (min(n_kv, p.n_past + kPrefillRows * (i + 1)) + kPrefillKeys - 1) / kPrefillKeys;
  };
  const int tA = tiles(qa);
  const int T = tA + (qz != qa ? tiles(qz) : 0);
  auto blk = [&](int u) { return u < tA ? qa : qz; };
  auto unit_tile = [&](int u) { return u < tA ? u : u - tA; };

  const int g = h / p.n_rep;
  const rsrc_t kr = make_rsrc(p.k + (int64_t)g * p.k_s1, (unsigned)((int64_t)(n_kv - 1) * p.k_s2 + D * ELT));
  const rsrc_t vr = make_rsrc(p.v + (int64_t)g * p.v_s1, (unsigned)((int64_t)(n_kv - 1) * p.v_s2 + D * ELT));
  const int ks2 = (int)p.k_s2, vs2 = (int)p.v_s2;

  // K tile of key tile kt into this wave's LDS tile: load i fills bytes
  // [1024 i, +1024), lane L its 16 bytes at 1024 i + 16 L, i.e. physical slot
  // pj of row r, which holds logical slot pj ^ swz(r). A tile wholly below
  // n_kv passes its row offset as the (unchecked) scalar offset; the tile that
  // crosses n_kv keeps it in the range-checked per-lane offset, so its rows
  // past n_kv arrive as zeros.
  lds_t* const ktile = lds + C::L_REG + wave * C::REG;
  unsigned koff[C::NDK];
#pragma unroll
  for (int i = 0; i < C::NDK; ++i) {
    const int o = 1024 * i + 16 * lane;
    const int r = o / C::RB;
    koff[i] = (unsigned)(r * ks2 + 16 * (((o % C::RB) / 16) ^ swz<NSLOT>(r)));
  }
  auto request_k = [&](int kt) __attribute__((always_inline)) {
    const int key0 = kt * kPrefillKeys;
    const unsigned to_lane = key0 + kPrefillKeys <= n_kv ? 0u : ~0u;
    const unsigned row = (unsigned)(key0 * ks2);
#pragma unroll
    for (int i = 0; i < C::NDK; ++i)
      dma16(kr, ktile + 1024 * i, koff[i] + (row & to_lane), row & ~to_lane);
  };
  // A operand of QK: K[key c][kh D/2 + s], s < D/2, from the LDS tile.
  auto read_k = [&](float (&kk)[HALF]) __attribute__((always_inline)) {
    const lds_t* const rowp = ktile + col * C::RB;
#pragma unroll
    for (int q = 0; q < C::HSL; ++q) {
      const lds_t* const a = rowp + 16 * ((kh * C::HSL + q) ^ swz<NSLOT>(col));
      if constexpr (ELT == 4) {
        const f32x4 x = *reinterpret_cast<const lds_f32x4*>(a);
        kk[4 * q + 0] = x[0]; kk[4 * q + 1] = x[1]; kk[4 * q + 2] = x[2]; kk[4 * q + 3] = x[3];
      } else {
        const f16x8 x = *reinterpret_cast<const lds_f16x8*>(a);
#pragma unroll
        for (int e = 0; e < 8; ++e) kk[8 * q + e] = (float)x[e];
      }
    }
  };
  // A operand of PV for key tile kt (rows past n_kv are zero, as for K):
  // lane (col, kh) holds V[key][NDB col + db] for the 16 keys 8 (t / 4) +
  // 4 kh + t % 4, one load of NDB consecutive elements per key. Output block
  // db's row c is therefore dim NDB c + db (write_record puts dims back in
  // order).
  const unsigned vvo = (unsigned)(4 * kh * vs2 + col * NDB * ELT);
  // key t's V values of key tile kt into vv[NDB t ..]
  auto load_v_key = [&](int kt, int t, float (&vv)[NV]) __attribute__((always_inline)) {
    const int key0 = kt * kPrefillKeys;
    const unsigned to_lane = key0 + kPrefillKeys <= n_kv ? 0u : ~0u;
    {
      const unsigned row = (unsigned)((key0 + 8 * (t >> 2) + (t & 3)) * vs2);
      const unsigned vo = vvo + (row & to_lane), so = row & ~to_lane;
      if constexpr (ELT == 4 && NDB == 2) {
        const f32x2 x = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(vr, vo, so, 0));
        vv[2 * t] = x[0];
        vv[2 * t + 1] = x[1];
      } else if constexpr (ELT == 4 && NDB == 4) {
        const f32x4 x = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, vo, so, 0));
#pragma unroll
        for (int db = 0; db < 4; ++db) vv[4 * t + db] = x[db];
      } else if constexpr (ELT == 2 && NDB == 2) {
        const f16x2 x = __builtin_bit_cast(f16x2, __builtin_amdgcn_raw_buffer_load_b32(vr, vo, so, 0));
        vv[2 * t] = (float)x[0];
        vv[2 * t + 1] = (float)x[1];
      } else {
        const f16x4 x = __builtin_bit_cast(f16x4, __builtin_amdgcn_raw_buffer_load_b64(vr, vo, so, 0));
#pragma unroll
        for (int db = 0; db < 4; ++db) vv[4 * t + db] = (float)x[db];
      }
    }
  };
  auto load_v = [&](int kt, float (&vv)[NV]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 16; ++t) load_v_key(kt, t, vv);
  };

  // The first unit of each wave is fixed (unit `wave`): its K tile is
  // requested before the workgroup's setup.
  if (wave < T) request_k(unit_tile(wave));

  // Setup: the unit counter (the next unit to take), block-qa records that are
  // never written keep m = -inf, and at head_dim 64 the pre-scaled queries of
  // both blocks.
  lds_u32* const ctr = (lds_u32*)(lds + C::L_CTR);
  auto rec_at = [&](int w, int slot) __attribute__((always_inline)) {
    return (lds_f32*)(lds + (slot == 0 ? C::L_REC0 + w * C::RECB : C::L_REG + w * C::REG));
  };
  if (threadIdx.x == 0) *ctr = (unsigned)NW;
  if (lane < kPrefillRows) rec_at(wave, 0)[kPrefillRows * RS + lane] = -INFINITY;
  if constexpr (C::QLDS) {
    constexpr int BQ4 = kPrefillRows * D / 4;  // float4 pieces of one block
#pragma unroll
    for (int i = threadIdx.x; i < 2 * BQ4; i += NW * kWave) {
      const int b = i / BQ4, row = (i % BQ4) / (D / 4), d4 = i % (D / 4);
      const int qloc = (b == 0 ? qa : qz) * kPrefillRows + row;
      const bool qvalid = qloc < p.n_tokens;
      // queries past n_tokens read row 0 (any finite row) and weigh zero
      const float4 v = *reinterpret_cast<const float4*>(
          reinterpret_cast<const char*>(p.q) + (int64_t)(qvalid ? qloc : 0) * p.q_s2 +
          (int64_t)h * p.q_s1 + 16 * d4);
      const float sc = qvalid ? p.scale_log2e : 0.f;
      *reinterpret_cast<lds_f32x4*>(lds + C::L_Q + ((b * kPrefillRows + row) * C::QRS + 4 * d4) * 4) =
          f32x4{v.x * sc, v.y * sc, v.z * sc, v.w * sc};
    }
  }
  __syncthreads();
  // The next unit: from the LDS counter, or (deterministic launches) the
  // wave's fixed sequence, so that which wave computes which unit, and with
  // it every rounding, is the same on every run: rounds of NW units, wave w
  // taking unit w of each, except that with two waves per SIMD (NW = 8) the
  // last round's units (when there is more than one round) go to the first
  // NW/2 waves, two each. The two waves of a SIMD share its matrix core and
  // the issue arbiter favours the older (the first NW/2): with equal shares
  // the younger finished its last units alone, 4 us after the older (n=1024;
  // moving them took 81.4 to 82.6 TFLOP/s). A unit index >= T means none.
  int seq = 0;  // index in the wave's sequence of the unit last taken
  const int det = __builtin_amdgcn_readfirstlane(p.det);
  constexpr int kShiftRounds = 1;  // (2 measured slower at n=1024, 80.2 against 82.7 TFLOP/s)
  const int last_round = (T - 1) / NW;
  const int shift0 = max(last_round - kShiftRounds + 1, 1);  // first shifted round
  auto take = [&]() __attribute__((always_inline)) {
    if (det) {
      ++seq;
      if (NW <= 4 || T <= NW || seq < shift0) return seq * NW + wave;
      if (wave >= NW / 2) return T;
      const int i = seq - shift0;  // the wave's i-th unit of the shifted rounds
      return i < 2 * (last_round - shift0 + 1) ? shift0 * NW + i * (NW / 2) + wave : T;
    }
    unsigned t = 0;
    if (lane == 0) t = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return __builtin_amdgcn_readfirstlane((int)t);
  };

  float qb[HALF];
  floatx16 o[NDB];
  float m = -INFINITY, lsum = 0.f;
  int cur = -1;  // query block of the running state

  // The block's queries (pre-scaled by scale*log2(e)) into qb.
  auto load_q = [&](int X) __attribute__((always_inline)) {
    if constexpr (C::QLDS) {
      const lds_t* const qp =
          lds + C::L_Q + (((X == qa ? 0 : 1) * kPrefillRows + col) * C::QRS + kh * HALF) * 4;
#pragma unroll
      for (int s = 0; s < HALF; s += 4) {
        const f32x4 v = *reinterpret_cast<const lds_f32x4*>(qp + 4 * s);
        qb[s + 0] = v[0]; qb[s + 1] = v[1]; qb[s + 2] = v[2]; qb[s + 3] = v[3];
      }
    } else {
      const int qloc = X * kPrefillRows + col;
      const bool qvalid = qloc < p.n_tokens;
      const float* qp = reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.q) +
                                                       (int64_t)(qvalid ? qloc : 0) * p.q_s2 +
                                                       (int64_t)h * p.q_s1) +
                        kh * HALF;
      const float sc = qvalid ? p.scale_log2e : 0.f;
#pragma unroll
      for (int s = 0; s < HALF; s += 4) {
        const float4 v = *reinterpret_cast<const float4*>(qp + s);
        qb[s + 0] = v.x * sc; qb[s + 1] = v.y * sc; qb[s + 2] = v.z * sc; qb[s + 3] = v.w * sc;
      }
    }
  };
  auto reset = [&](int X) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (floatx16)(0.f);
    m = -INFINITY;
    lsum = 0.f;
    cur = X;
  };

  // (m, l, O) of this wave's part of a block into its record.
  auto write_record = [&](int slot) __attribute__((always_inline)) {
    lds_f32* const rec = rec_at(wave, slot);
    const float ltot = xor32_sum(lsum);
    // register 4 r4 + i of block db holds dim NDB (8 r4 + 4 kh + i) + db
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          rec[col * RS + NDB * (8 * r4 + 4 * kh + i) + db] = o[db][4 * r4 + i];
    if (kh == 0) {
      rec[kPrefillRows * RS + col] = m;
      rec[kPrefillRows * RS + kPrefillRows + col] = ltot;
    }
  };

  // The block's queries as bf16 pairs (SPLIT), or f16 pairs with an F16
  // cache (F16P): step s, item i holds dim kh HALF + 8 s + i, the dims of
  // kk[8 s + i] (any pairing of the k-values is a valid contraction as long
  // as A and B agree). F16P: a wave whose largest |query| exceeds 2^14 takes
  // its queries times 2^-e (exact), so that their f16 pairs stay in range,
  // and its scores times 2^e.
  constexpr bool F16P = SPLIT && ELT == 2;
  typedef typename std::conditional<F16P, f16x8, bf16x8>::type qop_t;
  qop_t qh[SPLIT ? HALF / 8 : 1], ql[SPLIT ? HALF / 8 : 1];
  float qunscale = 1.f;
  auto split_q = [&]() __attribute__((always_inline)) {
    if constexpr (F16P) {
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < HALF; ++i) amax = fmaxf(amax, fabsf(qb[i]));
      amax = wave_max(amax);
      float f = 1.f;
      qunscale = 1.f;
      if (amax > 16384.f) {
        const int e = ilogbf(amax) - 13;
        f = ldexpf(1.f, -e);
        qunscale = ldexpf(1.f, e);
      }
#pragma unroll
      for (int st = 0; st < HALF / 8; ++st) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = qb[8 * st + i] * f;
        split8h(x, qh[st], ql[st]);
      }
    } else if constexpr (SPLIT) {
#pragma unroll
      for (int st = 0; st < HALF / 8; ++st) split8(qb + 8 * st, qh[st], ql[st]);
    }
  };

  // S^T = K . Q^T: D/2 v_mfma_f32_32x32x2f32, or (SPLIT) D/16 steps of three
  // v_mfma_f32_32x32x16_bf16 on bf16-pair-split operands
  auto qk = [&](const float (&kk)[HALF]) __attribute__((always_inline)) {
    floatx16 s = (floatx16)(0.f);
    if constexpr (F16P) {
#pragma unroll
      for (int st = 0; st < HALF / 8; ++st) {
        f16x8 k8;
        pack8h(kk + 8 * st, k8);
        s = mfma2h(k8, qh[st], ql[st], s);
      }
      if (qunscale != 1.f) s *= qunscale;
    } else if constexpr (SPLIT) {
#pragma unroll
      for (int st = 0; st < HALF / 8; ++st) {
        bf16x8 kh8, kl8;
        split8(kk + 8 * st, kh8, kl8);
        s = mfma3(kh8, kl8, qh[st], ql[st], s);
      }
    } else {
#pragma unroll
      for (int st = 0; st < HALF; ++st) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[st], qb[st], s, 0, 0, 0);
    }
    return s;
  };

  // Causal mask of unit (block X, tile kt), applied only where some key of
  // the tile lies past some query of the block (a wave-uniform test: the
  // diagonal tile, and tiles crossing n_kv, whose keys past n_kv are past
  // every query).
  auto mask = [&](floatx16& s, int X, int kt) __attribute__((always_inline)) {
    if (p.n_past + (X - kt) * kPrefillRows < kPrefillKeys - 1) {
      const int lim = p.n_past + X * kPrefillRows + col - kt * kPrefillKeys - 4 * kh;
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) s[rr] = 8 * (rr >> 2) + (rr & 3) > lim ? -INFINITY : s[rr];
    }
  };
  // Online softmax (base 2) of a masked unit: s becomes the probabilities,
  // (m, lsum) move on and alpha holds O's pending rescale factor. No
  // branches, so the next unit's QK products interleave with it.
  float alpha = 1.f;
  auto softmax = [&](floatx16& s) __attribute__((always_inline)) {
    const float a0 = fmaxf(fmaxf(s[0], s[1]), s[2]), a1 = fmaxf(fmaxf(s[3], s[4]), s[5]);
    const float a2 = fmaxf(fmaxf(s[6], s[7]), s[8]), a3 = fmaxf(fmaxf(s[9], s[10]), s[11]);
    const float a4 = fmaxf(fmaxf(s[12], s[13]), s[14]);
    const float mx = fmaxf(fmaxf(fmaxf(a0, a1), fmaxf(a2, a3)), fmaxf(a4, s[15]));
    const float mn = fmaxf(m, xor32_max(mx));
    const float mu = mn == -INFINITY ? 0.f : mn;
    alpha = fast_exp2(m - mu);
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) s[rr] = fast_exp2(s[rr] - mu);
    const float b0 = (s[0] + s[1]) + (s[2] + s[3]), b1 = (s[4] + s[5]) + (s[6] + s[7]);
    const float b2 = (s[8] + s[9]) + (s[10] + s[11]), b3 = (s[12] + s[13]) + (s[14] + s[15]);
    lsum = lsum * alpha + ((b0 + b1) + (b2 + b3));
    m = mn;
  };
  // O's rescale, skipped when no row's maximum moved (alpha == 1 throughout)
  auto rescale_o = [&]() __attribute__((always_inline)) {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0ull) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] *= alpha;
    }
  };

  // O^T += V^T . P^T: 16 v_mfma_f32_32x32x2f32 per 32 output dims, or (SPLIT)
  // two steps of three v_mfma_f32_32x32x16_bf16, step u taking registers
  // 8u .. 8u + 7 of S^T (keys 8 (r / 4) + 4 kh + r % 4) and the V values of
  // the same keys
  auto pv = [&](const floatx16& s, const float (&vv)[NV]) __attribute__((always_inline)) {
    if constexpr (F16P) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float pf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[i] = s[8 * u + i];
        f16x8 ph, pl;
        split8h(pf, ph, pl);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          float vf[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) vf[i] = vv[(8 * u + i) * NDB + db];
          f16x8 v8;
          pack8h(vf, v8);
          o[db] = mfma2h(v8, ph, pl, o[db]);
        }
      }
    } else if constexpr (SPLIT) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float pf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) pf[i] = s[8 * u + i];
        bf16x8 ph, pl;
        split8(pf, ph, pl);
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          float vf[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) vf[i] = vv[(8 * u + i) * NDB + db];
          bf16x8 vh, vl;
          split8(vf, vh, vl);
          o[db] = mfma3(vh, vl, ph, pl, o[db]);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < 16; ++t)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[t * NDB + db], s[t], o[db], 0, 0, 0);
    }
  };
  // Float products with an F32 cache: the PV products of one tile, each key's
  // V registers reloaded with key tile kt's values as soon as its products
  // have read them, so that the next unit's V has the rest of this PV and the
  // next QK to land behind (one buffer, the same 16 requests in key order).
  constexpr bool PV_INTERLEAVE = !SPLIT && ELT == 4;
  auto pv_load_v = [&](const floatx16& s, float (&vv)[NV], int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[t * NDB + db], s[t], o[db], 0, 0, 0);
      load_v_key(kt, t, vv);
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      __builtin_amdgcn_sched_group_barrier(0x008, NDB, 0);  // the key's MFMAs
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // then its V load
    }
  };

  // The wave's units, software-pipelined (see the header). Request order per
  // iteration: the next unit's K tile, then the current V loads; the wait
  // before reading a K tile allows the WAIT_K loads issued after it.
  float kk[HALF], vv[NV];
  floatx16 sc;
  int u = wave;
  if (u < T) {
    load_q(blk(u));
    split_q();
    reset(blk(u));
    wait_vmem<0>();
    read_k(kk);
    int un = take();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the tile is read before it is refilled
    if (un < T) request_k(unit_tile(un));
    __builtin_amdgcn_sched_barrier(0);
    // (after the K request: every K request is followed by exactly NVL loads
    // before the wait that reads its tile)
    load_v(unit_tile(u), vv);
    sc = qk(kk);
    while (un < T) {
      // sc: scores of unit u; the LDS tile is filling with unit un's K
      const int unn = take();
      const int Xu = blk(u), Xn = blk(un);
      if (Xn != Xu) {  // the running state still belongs to Xu
        load_q(Xn);
        split_q();
      }
      mask(sc, Xu, unit_tile(u));
      wait_vmem<C::WAIT_K>();
      read_k(kk);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the whole A operand at once
      // The tile is read: refill it with unit unn's K now, so that the load
      // has this iteration's products to land behind (no request past the
      // wave's last unit: its region becomes a record).
      if (unn < T) request_k(unit_tile(unn));
      __builtin_amdgcn_sched_barrier(0);
      const floatx16 sn = qk(kk);
      softmax(sc);
      if constexpr (!SPLIT) {
        // one QK product, then a few softmax instructions, in turn (the
        // products form a dependent chain that would otherwise stall the
        // wave's issue, the softmax waiting behind them)
#pragma unroll
        for (int i = 0; i < HALF; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      rescale_o();
      if constexpr (PV_INTERLEAVE) {
        pv_load_v(sc, vv, unit_tile(un));
      } else {
        pv(sc, vv);
      }
      if (Xn != Xu) {
        write_record(0);  // this wave's part of block qa
        reset(Xn);
      }
      if constexpr (!PV_INTERLEAVE) load_v(unit_tile(un), vv);
      sc = sn;
      u = un;
      un = unn;
    }
    // the last unit: no next QK to overlap
    mask(sc, blk(u), unit_tile(u));
    softmax(sc);
    rescale_o();
    pv(sc, vv);
    wait_vmem<0>();  // every load has landed before the region becomes a record
    write_record(cur == qa ? 0 : 1);
  }
  // a wave without a block-qz record marks its region (it held a K tile)
  if ((cur != qz || qz == qa) && lane < kPrefillRows) rec_at(wave, 1)[kPrefillRows * RS + lane] = -INFINITY;
  __syncthreads();

  // Merge: for each block, the waves that took part of it.
  constexpr int NQ4 = kPrefillRows * D / 4;  // (row, 4 dims) per block
#pragma unroll
  for (int slot = 0; slot < 2; ++slot) {
    if (slot == 1 && qz == qa) break;
    const int X = slot == 0 ? qa : qz;
    for (int idx = threadIdx.x; idx < NQ4; idx += NW * kWave) {
      const int row = idx / (D / 4), d4 = idx % (D / 4);
      if (X * kPrefillRows + row >= p.n_tokens) continue;
      float mx = -INFINITY;
      for (int w = 0; w < NW; ++w) mx = fmaxf(mx, rec_at(w, slot)[kPrefillRows * RS + row]);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      float l = 0.f;
      for (int w = 0; w < NW; ++w) {
        const lds_f32* const rec = rec_at(w, slot);
        const float mw = rec[kPrefillRows * RS + row];
        if (mw == -INFINITY) continue;  // a record the wave never wrote (any other m is finite)
        const float wt = fast_exp2(mw - mx);
        acc += wt * *reinterpret_cast<const lds_f32x4*>(rec + row * RS + 4 * d4);
        l += wt * rec[kPrefillRows * RS + kPrefillRows + row];
      }
      float* op = reinterpret_cast<float*>(reinterpret_cast<char*>(p.out) +
                                           (int64_t)(X * kPrefillRows + row) * p.o_s2 +
                                           (int64_t)h * p.o_s1);
      *reinterpret_cast<f32x4*>(op + 4 * d4) = acc * (1.f / l);
    }
  }
}

// Waves per workgroup: two per SIMD at head_dim 64, one at 128 (register budget).
template <int D>
constexpr int prefill_waves() {
  return D == 64 ? 8 : 4;
}

// Workgroups per head for a pairing (lone = 0 or 1).
static int prefill_wgs_per_head(int n_qblocks, int lone) {
  return lone + (n_qblocks - lone + 1) / 2;
}

// The pairing whose longest workgroup runs shortest: launch rounds on n_cu
// CUs times the units of the longest workgroup per SIMD (the matrix cores
// bound a unit; the waves of a workgroup share its CU's four SIMDs). At
// n_past = 0 pairs (j, NQ - 1 - j) give NQ + 1 units, the lone-last pairing
// NQ: with eight waves that is 8.25 against 8 units per SIMD.
static int prefill_choose_lone(const PrefillParams& p, int n_cu) {
  const int n_kv = p.n_past + p.n_tokens;
  auto tiles = [&](int i) {
    return (std::min(n_kv, p.n_past + kPrefillRows * (i + 1)) + kPrefillKeys - 1) / kPrefillKeys;
  };
  int64_t best = -1;
  int best_lone = 0;
  for (int lone = 0; lone <= (p.n_qblocks > 1 ? 1 : 0); ++lone) {
    const int per_head = prefill_wgs_per_head(p.n_qblocks, lone);
    int umax = 0;
    for (int j = 0; j < per_head; ++j) {
      const bool alone = lone && j == 0;
      const int qa = alone ? p.n_qblocks - 1 : j - lone;
      const int qz = alone ? qa : p.n_qblocks - 1 - lone - qa;
      umax = std::max(umax, tiles(qa) + (qz != qa ? tiles(qz) : 0));
    }
    const int64_t wgs = (int64_t)p.n_head * per_head;
    const int64_t cost = (wgs + n_cu - 1) / n_cu * ((umax + 3) / 4);
    if (best < 0 || cost < best) {
      best = cost;
      best_lone = lone;
    }
  }
  return best_lone;
}

template <int D, typename KT, bool SPLIT>
static hipError_t launch_prefill_t(PrefillParams p, int n_cu, hipStream_t stream) {
  constexpr int NW = prefill_waves<D>();
  typedef PrefillCfg<D, KT, NW> C;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<D, KT, NW, SPLIT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
  if (attr != hipSuccess) return attr;
  p.lone = prefill_choose_lone(p, n_cu);
  const unsigned per_head = (unsigned)prefill_wgs_per_head(p.n_qblocks, p.lone);
  hipLaunchKernelGGL((prefill_kernel<D, KT, NW, SPLIT>), dim3((unsigned)p.n_head * per_head),
                     dim3(NW * kWave), C::LDS, stream, p);
  return hipGetLastError();
}

template <int D, typename KT>
static hipError_t launch_prefill_m(const PrefillParams& p, int n_cu, bool split, hipStream_t stream) {
  return split ? launch_prefill_t<D, KT, true>(p, n_cu, stream) : launch_prefill_t<D, KT, false>(p, n_cu, stream);
}

hipError_t launch_prefill(const PrefillParams& p, int head_dim, bool f16, int n_cu, bool split,
                          hipStream_t stream) {
  if (head_dim == 64)
    return f16 ? launch_prefill_m<64, _Float16>(p, n_cu, split, stream)
               : launch_prefill_m<64, float>(p, n_cu, split, stream);
  if (head_dim == 128)
    return f16 ? launch_prefill_m<128, _Float16>(p, n_cu, split, stream)
               : launch_prefill_m<128, float>(p, n_cu, split, stream);
  return hipErrorInvalidValue;
}

}  // namespace mi
