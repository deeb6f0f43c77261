// prefill.hip -- fused causal ATTN_QK -> SOFTMAX -> ATTN_KQV for n_tokens > 1
// queries (src/ops_cpu.cpp:304-410), on the FP32 matrix cores of gfx950.
//
// One workgroup owns one (Q head h, block of 32 queries). Its waves take the
// block's visible key tiles (32 keys each) round-robin; each wave keeps a
// running (max, sum, O) per query and per tile
//   1. writes the tile's 32 K and V rows of KV head h / n_rep, prefetched into
//      registers during the previous tile, into its own padded LDS tiles
//      (F16 caches widen on the way), and issues the loads of its next tile;
//   2. computes S^T = K . Q^T (keys x queries) with D/2
//      v_mfma_f32_32x32x2f32: A = K rows from LDS, B = the block's queries,
//      pre-scaled by scale*log2(e) and held in registers for the whole block;
//   3. applies the causal mask (key > n_past + query) on tiles that reach the
//      diagonal, and the online softmax: a lane holds 16 keys of one query and
//      its partner lane (lane ^ 32) the other 16, so the row max is one
//      exchange and the exp2 is elementwise;
//   4. accumulates O^T += V^T . P^T with 16 MFMAs per 32 output dims. The
//      probabilities S^T leave step 3 in exactly the B-operand layout of this
//      product (register r of a lane = key 8(r/4) + 4(lane/32) + r%4), so no
//      shuffle or LDS round trip is needed.
// The waves then merge their (m, l, O) through LDS with the stable rescaling
// and write the block's output; nothing leaves the workgroup but the result.
// Workgroups are numbered from the longest query block down so long blocks
// start first, and the heads of one block are adjacent so K/V tiles of a
// shared KV head are re-read from L2.
#include "attn_common.h"
#include "kernels.h"

namespace mi {

typedef float floatx16 __attribute__((ext_vector_type(16)));

template <int D, typename KT>
__global__ __launch_bounds__(kPrefillWaves* kWave) void prefill_kernel(const PrefillParams p) {
  constexpr int ELT = (int)sizeof(KT);
  constexpr int KS = D + 4;                 // LDS K row stride (floats)
  constexpr int VS = D + 8;                 // LDS V row stride (floats)
  constexpr int HALF = D / 2;               // QK MFMA steps
  constexpr int NDB = D / 32;               // PV output blocks of 32 dims
  constexpr int LPR = D / 4;                // staging: lanes per row
  constexpr int RPI = kWave / LPR;          // staging: rows per instruction
  constexpr int NLD = kPrefillKeys / RPI;   // staging: instructions per tile
  constexpr int WS = kPrefillKeys * (KS + VS);
  constexpr int RS = kPrefillRows * D + 2 * kPrefillRows;  // merge record
  static_assert(RS <= WS, "merge record must fit the wave's staging area");

  extern __shared__ float lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  float* kl = lds + wave * WS;
  float* vl = kl + kPrefillKeys * KS;

  // workgroup -> (head h, query block i), longest blocks first
  const int h = blockIdx.x % p.n_head;
  const int i = p.n_qblocks - 1 - (int)(blockIdx.x / p.n_head);
  const int n_kv = p.n_past + p.n_tokens;
  const int q_first = i * kPrefillRows;
  const int kt_i = (min(n_kv, p.n_past + q_first + kPrefillRows) + kPrefillKeys - 1) / kPrefillKeys;

  const int g = h / p.n_rep;
  const int col = lane & 31;  // query row in B / key row in A
  const int kh = lane >> 5;
  const int qloc = q_first + col;
  const bool qvalid = qloc < p.n_tokens;
  const int qabs = p.n_past + qloc;

  float qb[HALF];
  {
    const float* qp = reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.q) +
                                                     (int64_t)qloc * p.q_s2 +
                                                     (int64_t)h * p.q_s1) +
                      kh * HALF;
#pragma unroll
    for (int s = 0; s < HALF; s += 4) {
      const float4 v = qvalid ? *reinterpret_cast<const float4*>(qp + s)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
      qb[s + 0] = v.x * p.scale_log2e;
      qb[s + 1] = v.y * p.scale_log2e;
      qb[s + 2] = v.z * p.scale_log2e;
      qb[s + 3] = v.w * p.scale_log2e;
    }
  }

  floatx16 o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = (floatx16)(0.f);
  float m = -INFINITY, lsum = 0.f;

  const char* kb = p.k + (int64_t)g * p.k_s1;
  const char* vb = p.v + (int64_t)g * p.v_s1;
  const int sr = lane / LPR, sc4 = lane % LPR;
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);

  // K/V rows of tile kt into registers (rows past n_kv read as zero).
  float4 kr[NLD], vr[NLD];
  auto fetch = [&](int kt) {
    const int key0 = kt * kPrefillKeys;
    const int kvalid = min(kPrefillKeys, n_kv - key0);
#pragma unroll
    for (int li = 0; li < NLD; ++li) {
      const int row = li * RPI + sr;
      const bool ok = row < kvalid;
      kr[li] = ok ? load4<KT>(kb + (int64_t)(key0 + row) * p.k_s2 + sc4 * 4 * ELT) : zero4;
      vr[li] = ok ? load4<KT>(vb + (int64_t)(key0 + row) * p.v_s2 + sc4 * 4 * ELT) : zero4;
    }
  };

  if (wave < kt_i) fetch(wave);
  for (int kt = wave; kt < kt_i; kt += nwaves) {
    const int key0 = kt * kPrefillKeys;
    wave_lds_fence();
#pragma unroll
    for (int li = 0; li < NLD; ++li) {
      const int row = li * RPI + sr;
      *reinterpret_cast<float4*>(&kl[row * KS + sc4 * 4]) = kr[li];
      *reinterpret_cast<float4*>(&vl[row * VS + sc4 * 4]) = vr[li];
    }
    wave_lds_fence();
    if (kt + nwaves < kt_i) fetch(kt + nwaves);  // in flight during this tile

    // S^T = K . Q^T
    floatx16 s = (floatx16)(0.f);
    const float* ka = kl + col * KS + kh * HALF;
#pragma unroll
    for (int st = 0; st < HALF; st += 4) {
      const float4 a = *reinterpret_cast<const float4*>(ka + st);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, qb[st + 0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, qb[st + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, qb[st + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, qb[st + 3], s, 0, 0, 0);
    }

    // Causal mask and online softmax (base 2).
    const bool diag = key0 + kPrefillKeys - 1 > p.n_past + q_first;
    float mx = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      float x = s[rr];
      if (diag) {
        const int key = key0 + 8 * (rr >> 2) + 4 * kh + (rr & 3);
        if (key > qabs) x = -INFINITY;
      }
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
    for (int t = 0; t < 16; ++t) {
      const int keyl = 8 * (t >> 2) + 4 * kh + (t & 3);
      const float* va = vl + keyl * VS + col;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[db * 32], s[t], o[db], 0, 0, 0);
    }
  }

  // Merge the waves through LDS: record = [32 rows][D] O, m[32], l[32].
  const float ltot = lsum + __shfl_xor(lsum, 32, kWave);
  wave_lds_fence();
  float* rec = kl;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      *reinterpret_cast<float4*>(rec + col * D + 32 * db + 8 * r4 + 4 * kh) =
          make_float4(o[db][4 * r4 + 0], o[db][4 * r4 + 1], o[db][4 * r4 + 2], o[db][4 * r4 + 3]);
  if (kh == 0) {
    rec[kPrefillRows * D + col] = m;
    rec[kPrefillRows * D + kPrefillRows + col] = ltot;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < kPrefillRows * D; idx += blockDim.x) {
    const int row = idx / D, d = idx % D;
    if (q_first + row >= p.n_tokens) continue;
    float mx = -INFINITY;
    for (int w = 0; w < nwaves; ++w) mx = fmaxf(mx, lds[w * WS + kPrefillRows * D + row]);
    float a = 0.f, l = 0.f;
    for (int w = 0; w < nwaves; ++w) {
      const float* r = lds + w * WS;
      const float wt = fast_exp2(r[kPrefillRows * D + row] - mx);  // idle wave: -inf -> 0
      a += wt * r[row * D + d];
      l += wt * r[kPrefillRows * D + kPrefillRows + row];
    }
    float* op = reinterpret_cast<float*>(reinterpret_cast<char*>(p.out) +
                                         (int64_t)(q_first + row) * p.o_s2 + (int64_t)h * p.o_s1);
    op[d] = a / l;
  }
}

template <int D, typename KT>
static hipError_t launch_prefill_t(const PrefillParams& p, hipStream_t stream) {
  constexpr int WS = kPrefillKeys * ((D + 4) + (D + 8));
  const size_t lds = (size_t)kPrefillWaves * WS * sizeof(float);
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<D, KT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((prefill_kernel<D, KT>), dim3((unsigned)(p.n_head * p.n_qblocks)),
                     dim3(kPrefillWaves * kWave), lds, stream, p);
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
