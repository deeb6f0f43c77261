// prefill.hip -- fused causal ATTN_QK -> SOFTMAX -> ATTN_KQV for n_tokens > 1
// queries (src/ops_cpu.cpp:304-410), on the FP32 matrix cores of gfx950.
//
// Work decomposition. A query block is 32 consecutive queries of one head; it
// sees ceil((n_past + 32 (i + 1)) / 32) key tiles of 32 keys (causal). One
// workgroup owns the query blocks i and NQ - 1 - i of one head, so every
// workgroup has the same number of tiles (NQ + 1 + 2 n_past / 32 when the
// blocks are full). Its NW waves cut that list of (block, tile) units into
// equal contiguous ranges; a range crosses from block i to block NQ - 1 - i at
// most once, where the wave parks its first block's partial result in LDS.
//
// Per unit (lane = (c = lane % 32, kh = lane / 32)):
//   1. the tile's K rows and V columns come straight from memory (L2) into
//      registers in the matrix-core operand layouts: lane (c, kh) holds
//      K[key c][kh D/2 ..] and V[key][dim c + 32 db] for the 16 keys
//      8(t/4) + 4kh + t%4; K is requested one unit ahead, V at the start of
//      its unit, under the QK products;
//   2. S^T = K . Q^T with D/2 v_mfma_f32_32x32x2f32: A = K, B = the block's
//      queries, pre-scaled by scale*log2(e) and held in registers;
//   3. causal mask (key > n_past + query) on tiles that reach the diagonal,
//      online softmax in base 2: a lane holds 16 keys of query c and its
//      partner lane (lane ^ 32) the other 16 (one permlane32 swap combines
//      them); O is rescaled only in units where a running max moved;
//   4. O^T += V^T . P^T with 16 MFMAs per 32 output dims; S^T leaves step 3 in
//      the B-operand layout of this product (register r of a lane = key
//      8(r/4) + 4kh + r%4), so P needs no shuffle.
// At the end the waves' (m, l, O) records meet in LDS and each block's
// output is merged with the stable rescaling; nothing else leaves the
// workgroup. Two waves per SIMD at head_dim 64 (one at 128) let one wave's
// softmax and loads run under the other's matrix-core work.
#include "attn_common.h"
#include "kernels.h"

namespace mi {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

namespace {

// Descriptor over [p, p + bytes) (raw, unswizzled): loads at offsets >= bytes
// return zero.
__device__ inline rsrc_t prefill_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <typename KT>
struct Elt;
// Loads at byte offset vo (per lane) + so (wave-uniform, a scalar register);
// only vo (with the instruction's constant offset) is range-checked.
template <>
struct Elt<float> {
  // 4 consecutive elements
  __device__ static void load4(rsrc_t r, unsigned vo, unsigned so, float* d) {
    const f32x4 x = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
    d[0] = x[0]; d[1] = x[1]; d[2] = x[2]; d[3] = x[3];
  }
  __device__ static float load1(rsrc_t r, unsigned vo, unsigned so) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0));
  }
};
template <>
struct Elt<_Float16> {
  // 8 consecutive elements, widened exactly
  __device__ static void load8(rsrc_t r, unsigned vo, unsigned so, float* d) {
    const f16x8 x = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = (float)x[i];
  }
  __device__ static float load1(rsrc_t r, unsigned vo, unsigned so) {
    return (float)__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0));
  }
};

// x and lane ^ 32's x, in some order, in one v_permlane32_swap (no LDS round
// trip): swapping the upper half of one copy of x with the lower half of
// another leaves each lane holding both. Written as asm: the compiler's
// builtin for this instruction drops one of its two results when they are
// used as floats. The s_nop gives the two wait states a VALU write of an
// operand needs before the swap reads it.
__device__ inline void xor32_pair(float x, float& a, float& b) {
  float y = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
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

}  // namespace

template <int D, typename KT, int NW>
struct PrefillCfg {
  static constexpr int ELT = (int)sizeof(KT);
  static constexpr int HALF = D / 2;                        // QK MFMA steps
  static constexpr int NDB = D / 32;                        // PV output blocks of 32 dims
  static constexpr int NV = 16 * NDB;                       // V values per lane per tile
  static constexpr int RS = D + 4;                          // record row stride (floats)
  static constexpr int RECF = kPrefillRows * RS + 2 * kPrefillRows;  // O rows, m, l
  static constexpr int LDS = NW * 2 * RECF * 4;             // a record per (wave, block)
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int D, typename KT, int NW>
__global__ __launch_bounds__(NW* kWave) void prefill_kernel(const PrefillParams p) {
  typedef PrefillCfg<D, KT, NW> C;
  constexpr int HALF = C::HALF, NDB = C::NDB, NV = C::NV, RS = C::RS, ELT = C::ELT;

  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int col = lane & 31;
  const int kh = lane >> 5;

  // workgroup -> (head h, query blocks qa and qz)
  const int h = blockIdx.x % p.n_head;
  const int qa = blockIdx.x / p.n_head;
  const int qz = p.n_qblocks - 1 - qa;
  const int n_kv = p.n_past + p.n_tokens;
  auto tiles = [&](int i) {
    return (min(n_kv, p.n_past + kPrefillRows * (i + 1)) + kPrefillKeys - 1) / kPrefillKeys;
  };
  const int tA = tiles(qa);
  const int T = tA + (qz != qa ? tiles(qz) : 0);
  auto first_unit = [&](int w) { return T * w / NW; };
  const int u0 = first_unit(wave), u1 = first_unit(wave + 1);

  const int g = h / p.n_rep;
  const rsrc_t kr = prefill_rsrc(p.k + (int64_t)g * p.k_s1, (unsigned)((int64_t)(n_kv - 1) * p.k_s2 + D * ELT));
  const rsrc_t vr = prefill_rsrc(p.v + (int64_t)g * p.v_s1, (unsigned)((int64_t)(n_kv - 1) * p.v_s2 + D * ELT));
  const int ks2 = (int)p.k_s2, vs2 = (int)p.v_s2;

  // K and V of key tile kt in this lane's operand layouts. The buffer range
  // check covers the per-lane offset (and the instruction's constant), not the
  // scalar one: a tile wholly below n_kv moves its wave-uniform row offsets to
  // the scalar operand; the tile that crosses n_kv keeps the whole offset per
  // lane, so its rows past n_kv read as zero.
  const unsigned kvo = (unsigned)(col * ks2 + kh * HALF * ELT);
  const unsigned vvo = (unsigned)(4 * kh * vs2 + col * ELT);
  auto load_k = [&](int kt, float (&kk)[HALF]) __attribute__((always_inline)) {
    const int key0 = kt * kPrefillKeys;
    const bool whole = key0 + kPrefillKeys <= n_kv;
    const unsigned so = whole ? (unsigned)(key0 * ks2) : 0u;
    const unsigned vo = whole ? kvo : kvo + (unsigned)(key0 * ks2);
    if constexpr (ELT == 4) {
#pragma unroll
      for (int s = 0; s < HALF; s += 4) Elt<float>::load4(kr, vo + 4 * s, so, kk + s);
    } else {
#pragma unroll
      for (int s = 0; s < HALF; s += 8) Elt<_Float16>::load8(kr, vo + 2 * s, so, kk + s);
    }
  };
  auto load_v = [&](int kt, float (&vv)[NV]) __attribute__((always_inline)) {
    const int key0 = kt * kPrefillKeys;
    if (key0 + kPrefillKeys <= n_kv) {
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const unsigned so = (unsigned)((key0 + 8 * (t >> 2) + (t & 3)) * vs2);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          vv[t * NDB + db] = Elt<KT>::load1(vr, vvo + 32 * db * ELT, so);
      }
    } else {
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const unsigned vo = vvo + (unsigned)((key0 + 8 * (t >> 2) + (t & 3)) * vs2);
#pragma unroll
        for (int db = 0; db < NDB; ++db) vv[t * NDB + db] = Elt<KT>::load1(vr, vo + 32 * db * ELT, 0u);
      }
    }
  };
  auto unit_tile = [&](int u) { return u < tA ? u : u - tA; };

  float qb[HALF];
  floatx16 o[NDB];
  float m = -INFINITY, lsum = 0.f;
  int cur = -1;  // query block of the running state

  auto write_record = [&](int slot) __attribute__((always_inline)) {
    float* rec = lds + (wave * 2 + slot) * C::RECF;
    const float ltot = xor32_sum(lsum);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<f32x4*>(rec + col * RS + 32 * db + 8 * r4 + 4 * kh) =
            f32x4{o[db][4 * r4 + 0], o[db][4 * r4 + 1], o[db][4 * r4 + 2], o[db][4 * r4 + 3]};
    if (kh == 0) {
      rec[kPrefillRows * RS + col] = m;
      rec[kPrefillRows * RS + kPrefillRows + col] = ltot;
    }
  };

  auto start_block = [&](int X) __attribute__((always_inline)) {
    const int qloc = X * kPrefillRows + col;
    const bool qvalid = qloc < p.n_tokens;
    const float* qp = reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.q) +
                                                     (int64_t)(qvalid ? qloc : 0) * p.q_s2 +
                                                     (int64_t)h * p.q_s1) +
                      kh * HALF;
    // queries past n_tokens read row 0 (any finite row) and weigh zero
    const float sc = qvalid ? p.scale_log2e : 0.f;
#pragma unroll
    for (int s = 0; s < HALF; s += 4) {
      const float4 v = *reinterpret_cast<const float4*>(qp + s);
      qb[s + 0] = v.x * sc;
      qb[s + 1] = v.y * sc;
      qb[s + 2] = v.z * sc;
      qb[s + 3] = v.w * sc;
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (floatx16)(0.f);
    m = -INFINITY;
    lsum = 0.f;
    cur = X;
  };

  // Unit u with its K in kk: requests its V and the next unit's K (into kn)
  // before the QK products that hide them.
  auto step = [&](int u, const float (&kk)[HALF], float (&kn)[HALF]) __attribute__((always_inline)) {
    const int X = u < tA ? qa : qz;
    const int kt = u < tA ? u : u - tA;
    if (X != cur) {
      if (cur >= 0) write_record(0);  // the first block's part of this wave's range
      start_block(X);
    }
    float vv[NV];
    load_v(kt, vv);
    if (u + 1 < u1) load_k(unit_tile(u + 1), kn);

    // S^T = K . Q^T
    floatx16 s = (floatx16)(0.f);
#pragma unroll
    for (int st = 0; st < HALF; ++st) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[st], qb[st], s, 0, 0, 0);

    // Causal mask and online softmax (base 2).
    const int key0 = kt * kPrefillKeys;
    const int qabs = p.n_past + X * kPrefillRows + col;
    const bool diag = key0 + kPrefillKeys - 1 > p.n_past + X * kPrefillRows;
    if (diag) {
#pragma unroll
      for (int rr = 0; rr < 16; ++rr)
        if (key0 + 8 * (rr >> 2) + 4 * kh + (rr & 3) > qabs) s[rr] = -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int rr = 1; rr < 16; ++rr) mx = fmaxf(mx, s[rr]);
    const float mn = fmaxf(m, xor32_max(mx));
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = fast_exp2(m - mu);
    float ps = 0.f;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float e = fast_exp2(s[rr] - mu);
      s[rr] = e;
      ps += e;
    }
    lsum = lsum * alpha + ps;
    // O is rescaled only when some query's running max moved (alpha == 1 for
    // the others, exactly).
    if (__builtin_amdgcn_ballot_w64(mn != m)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] *= alpha;
    }
    m = mn;

    // O^T += V^T . P^T
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[t * NDB + db], s[t], o[db], 0, 0, 0);
  };

  // The range; K alternates between two register sets.
  float ka[HALF], kb[HALF];
  if (u0 < u1) load_k(unit_tile(u0), ka);
  for (int u = u0; u < u1; u += 2) {
    step(u, ka, kb);
    if (u + 1 >= u1) break;
    step(u + 1, kb, ka);
  }
  if (cur >= 0) write_record(cur == qa ? 0 : 1);
  __syncthreads();

  // Merge: for each block, the waves whose ranges touched it.
  constexpr int NQ4 = kPrefillRows * D / 4;  // (row, 4 dims) per block
#pragma unroll
  for (int slot = 0; slot < 2; ++slot) {
    if (slot == 1 && qz == qa) break;
    const int X = slot == 0 ? qa : qz;
    for (int idx = threadIdx.x; idx < NQ4; idx += NW * kWave) {
      const int row = idx / (D / 4), d4 = idx % (D / 4);
      if (X * kPrefillRows + row >= p.n_tokens) continue;
      float mx = -INFINITY;
      for (int w = 0; w < NW; ++w) {
        const int a = first_unit(w), b = first_unit(w + 1);
        const bool touched = slot == 0 ? a < min(b, tA) : max(a, tA) < b;
        if (touched) mx = fmaxf(mx, lds[(w * 2 + slot) * C::RECF + kPrefillRows * RS + row]);
      }
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      float l = 0.f;
      for (int w = 0; w < NW; ++w) {
        const int a = first_unit(w), b = first_unit(w + 1);
        const bool touched = slot == 0 ? a < min(b, tA) : max(a, tA) < b;
        if (!touched) continue;
        const float* rec = lds + (w * 2 + slot) * C::RECF;
        const float mw = rec[kPrefillRows * RS + row];
        const float wt = mw == -INFINITY ? 0.f : fast_exp2(mw - mx);
        acc += wt * *reinterpret_cast<const f32x4*>(rec + row * RS + 4 * d4);
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

template <int D, typename KT>
static hipError_t launch_prefill_t(const PrefillParams& p, hipStream_t stream) {
  constexpr int NW = prefill_waves<D>();
  typedef PrefillCfg<D, KT, NW> C;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<D, KT, NW>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
  if (attr != hipSuccess) return attr;
  const unsigned n_pairs = (unsigned)((p.n_qblocks + 1) / 2);
  hipLaunchKernelGGL((prefill_kernel<D, KT, NW>), dim3((unsigned)p.n_head * n_pairs),
                     dim3(NW * kWave), C::LDS, stream, p);
  return hipGetLastError();
}

hipError_t launch_prefill(const PrefillParams& p, int head_dim, bool f16, hipStream_t stream) {
  if (head_dim == 64)
    return f16 ? launch_prefill_t<64, _Float16>(p, stream) : launch_prefill_t<64, float>(p, stream);
  if (head_dim == 128)
    return f16 ? launch_prefill_t<128, _Float16>(p, stream)
               : launch_prefill_t<128, float>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace mi
