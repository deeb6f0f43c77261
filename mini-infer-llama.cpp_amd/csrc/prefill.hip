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
//      partner lane (lane ^ 32) the other 16;
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
template <>
struct Elt<float> {
  // 4 consecutive elements at byte offset o
  __device__ static void load4(rsrc_t r, unsigned o, float* d) {
    const f32x4 x = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0));
    d[0] = x[0]; d[1] = x[1]; d[2] = x[2]; d[3] = x[3];
  }
  __device__ static float load1(rsrc_t r, unsigned o) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0));
  }
};
template <>
struct Elt<_Float16> {
  // 8 consecutive elements at byte offset o, widened exactly
  __device__ static void load8(rsrc_t r, unsigned o, float* d) {
    const f16x8 x = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0));
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = (float)x[i];
  }
  __device__ static float load1(rsrc_t r, unsigned o) {
    return (float)__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(r, o, 0, 0));
  }
};

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

  // K and V of key tile kt in this lane's operand layouts (rows past n_kv are zero).
  auto load_k = [&](int kt, float (&kk)[HALF]) __attribute__((always_inline)) {
    const unsigned ko = (unsigned)((kt * kPrefillKeys + col) * ks2 + kh * HALF * ELT);
    if constexpr (ELT == 4) {
#pragma unroll
      for (int s = 0; s < HALF; s += 4) Elt<float>::load4(kr, ko + 4 * s, kk + s);
    } else {
#pragma unroll
      for (int s = 0; s < HALF; s += 8) Elt<_Float16>::load8(kr, ko + 2 * s, kk + s);
    }
  };
  auto load_v = [&](int kt, float (&vv)[NV]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const unsigned vo =
          (unsigned)((kt * kPrefillKeys + 8 * (t >> 2) + 4 * kh + (t & 3)) * vs2 + col * ELT);
#pragma unroll
      for (int db = 0; db < NDB; ++db) vv[t * NDB + db] = Elt<KT>::load1(vr, vo + 32 * db * ELT);
    }
  };
  auto unit_tile = [&](int u) { return u < tA ? u : u - tA; };

  float qb[HALF];
  floatx16 o[NDB];
  float m = -INFINITY, lsum = 0.f;
  int cur = -1;  // query block of the running state

  auto write_record = [&](int slot) __attribute__((always_inline)) {
    float* rec = lds + (wave * 2 + slot) * C::RECF;
    const float ltot = lsum + __shfl_xor(lsum, 32, kWave);
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
#pragma unroll
    for (int s = 0; s < HALF; s += 4) {
      const float4 v = *reinterpret_cast<const float4*>(qp + s);
      qb[s + 0] = qvalid ? v.x * p.scale_log2e : 0.f;
      qb[s + 1] = qvalid ? v.y * p.scale_log2e : 0.f;
      qb[s + 2] = qvalid ? v.z * p.scale_log2e : 0.f;
      qb[s + 3] = qvalid ? v.w * p.scale_log2e : 0.f;
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (floatx16)(0.f);
    m = -INFINITY;
    lsum = 0.f;
    cur = X;
  };

  // Unit u with its K in kk; requests its V and the next unit's K (into kn)
  // before the matrix-core work that hides them.
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
    float mx = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      float x = s[rr];
      if (diag && key0 + 8 * (rr >> 2) + 4 * kh + (rr & 3) > qabs) x = -INFINITY;
      s[rr] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float mn = fmaxf(m, mx);
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
    m = mn;
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] *= alpha;

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
