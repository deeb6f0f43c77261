// prefill.hip -- fused causal ATTN_QK -> SOFTMAX -> ATTN_KQV for n_tokens > 1
// queries (src/ops_cpu.cpp:304-410), on the FP32 matrix cores of gfx950.
//
// A wave owns one unit = (Q head h, block of 32 queries, chunk of C key
// tiles of 32 keys); units never share LDS, so a workgroup's waves never
// wait for each other. Per key tile the wave
//   1. stages the 32 K and V rows of KV head h / n_rep into its own padded
//      LDS tiles (coalesced 16-byte loads; F16 caches widen here);
//   2. computes S^T = K . Q^T (keys x queries) with D/2
//      v_mfma_f32_32x32x2f32: A = K rows from LDS, B = the wave's queries,
//      pre-scaled by scale*log2(e) and held in registers for the whole unit;
//   3. applies the causal mask (key > n_past + query) on tiles that reach the
//      diagonal, and the online softmax: a lane holds 16 keys of one query and
//      its partner lane (lane ^ 32) the other 16, so the row max is one
//      exchange and the exp2 is elementwise;
//   4. accumulates O^T += V^T . P^T with 16 MFMAs per 32 output dims. The
//      probabilities S^T leave step 3 in exactly the B-operand layout of this
//      product (register r of a lane = key 8(r/4) + 4(lane/32) + r%4), so no
//      shuffle or LDS round trip is needed.
// Queries whose visible keys span several chunks write (m, l, O) partials;
// the last of those units to arrive (device-scope counter per head and
// query block) merges them and resets the counter. Units are numbered from
// the longest query block down, so long units start first.
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
  constexpr int REC = kPrefillRows * (D + 2);

  extern __shared__ float lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int unit = blockIdx.x * (blockDim.x / kWave) + wave;
  if (unit >= p.n_units) return;

  float* kl = lds + wave * WS;
  float* vl = kl + kPrefillKeys * KS;

  // unit -> (head h, query block i, key chunk j)
  const int h = unit % p.n_head;
  const int r = p.units_per_head - 1 - unit / p.n_head;
  const int n_kv = p.n_past + p.n_tokens;
  const int kt_all = (n_kv + kPrefillKeys - 1) / kPrefillKeys;
  const int c0 = (p.n_past + kPrefillKeys - 1) / kPrefillKeys;
  const int C = p.chunk_tiles;
  const int64_t base = ceil_prefix(c0, C);
  int lo_i = 0, hi_i = p.n_qblocks - 1;
  while (lo_i < hi_i) {
    const int mid = (lo_i + hi_i + 1) / 2;
    if (ceil_prefix(c0 + mid, C) - base <= r)
      lo_i = mid;
    else
      hi_i = mid - 1;
  }
  const int i = lo_i;
  const int64_t f_i = ceil_prefix(c0 + i, C) - base;
  const int j = r - (int)f_i;
  const int kt_i = min(c0 + i + 1, kt_all);
  const int nch = (kt_i + C - 1) / C;
  const int t0 = j * C, t1 = min(t0 + C, kt_i);

  const int g = h / p.n_rep;
  const int col = lane & 31;  // query row in B / key row in A
  const int kh = lane >> 5;
  const int q_first = i * kPrefillRows;
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

  for (int kt = t0; kt < t1; ++kt) {
    const int key0 = kt * kPrefillKeys;
    const int kvalid = min(kPrefillKeys, n_kv - key0);
    float4 kr[NLD], vr[NLD];
#pragma unroll
    for (int li = 0; li < NLD; ++li) {
      const int row = li * RPI + sr;
      const bool ok = row < kvalid;
      kr[li] = ok ? load4<KT>(kb + (int64_t)(key0 + row) * p.k_s2 + sc4 * 4 * ELT) : zero4;
      vr[li] = ok ? load4<KT>(vb + (int64_t)(key0 + row) * p.v_s2 + sc4 * 4 * ELT) : zero4;
    }
    wave_lds_fence();
#pragma unroll
    for (int li = 0; li < NLD; ++li) {
      const int row = li * RPI + sr;
      *reinterpret_cast<float4*>(&kl[row * KS + sc4 * 4]) = kr[li];
      *reinterpret_cast<float4*>(&vl[row * VS + sc4 * 4]) = vr[li];
    }
    wave_lds_fence();

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
    wave_lds_fence();
  }

  const float ltot = lsum + __shfl_xor(lsum, 32, kWave);

  if (nch == 1) {
    if (qvalid) {
      const float inv = 1.f / ltot;
      float* op = reinterpret_cast<float*>(reinterpret_cast<char*>(p.out) +
                                           (int64_t)qloc * p.o_s2 + (int64_t)h * p.o_s1);
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(op + 32 * db + 8 * r4 + 4 * kh) =
              make_float4(o[db][4 * r4 + 0] * inv, o[db][4 * r4 + 1] * inv,
                          o[db][4 * r4 + 2] * inv, o[db][4 * r4 + 3] * inv);
    }
    return;
  }

  // Partial of this chunk: [32 rows][D] unnormalised O, then m[32], l[32].
  float* rec = p.part + ((f_i + j) * p.n_head + h) * REC;
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
  __threadfence();
  unsigned prev = 0;
  if (lane == 0) prev = atomicAdd(&p.counter[h * p.n_qblocks + i], 1u);
  prev = __shfl(prev, 0, kWave);
  if (prev != (unsigned)(nch - 1)) return;
  __threadfence();

  // Last chunk to arrive: merge the nch partials of (h, i).
  float mx = -INFINITY;
  for (int jj = 0; jj < nch; ++jj) {
    const float* rj = p.part + ((f_i + jj) * p.n_head + h) * REC;
    mx = fmaxf(mx, rj[kPrefillRows * D + col]);
  }
  float acc[HALF];
#pragma unroll
  for (int d = 0; d < HALF; ++d) acc[d] = 0.f;
  float total = 0.f;
  for (int jj = 0; jj < nch; ++jj) {
    const float* rj = p.part + ((f_i + jj) * p.n_head + h) * REC;
    const float w = fast_exp2(rj[kPrefillRows * D + col] - mx);
    total += w * rj[kPrefillRows * D + kPrefillRows + col];
#pragma unroll
    for (int d = 0; d < HALF; d += 4) {
      const float4 a = *reinterpret_cast<const float4*>(rj + col * D + kh * HALF + d);
      acc[d + 0] += w * a.x;
      acc[d + 1] += w * a.y;
      acc[d + 2] += w * a.z;
      acc[d + 3] += w * a.w;
    }
  }
  if (qvalid) {
    const float inv = 1.f / total;
    float* op = reinterpret_cast<float*>(reinterpret_cast<char*>(p.out) +
                                         (int64_t)qloc * p.o_s2 + (int64_t)h * p.o_s1) +
                kh * HALF;
#pragma unroll
    for (int d = 0; d < HALF; d += 4)
      *reinterpret_cast<float4*>(op + d) =
          make_float4(acc[d] * inv, acc[d + 1] * inv, acc[d + 2] * inv, acc[d + 3] * inv);
  }
  if (lane == 0) p.counter[h * p.n_qblocks + i] = 0u;
}

template <int D, typename KT>
static hipError_t launch_prefill_t(const PrefillParams& p, hipStream_t stream) {
  constexpr int WS = kPrefillKeys * ((D + 4) + (D + 8));
  const size_t lds = (size_t)kPrefillWaves * WS * sizeof(float);
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_kernel<D, KT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const unsigned blocks = (unsigned)((p.n_units + kPrefillWaves - 1) / kPrefillWaves);
  hipLaunchKernelGGL((prefill_kernel<D, KT>), dim3(blocks), dim3(kPrefillWaves * kWave), lds,
                     stream, p);
  return hipGetLastError();
}

size_t prefill_record_floats(int head_dim) { return (size_t)kPrefillRows * (head_dim + 2); }

hipError_t launch_prefill(const PrefillParams& p, int head_dim, bool f16, hipStream_t stream) {
  if (head_dim == 64)
    return f16 ? launch_prefill_t<64, _Float16>(p, stream) : launch_prefill_t<64, float>(p, stream);
  if (head_dim == 128)
    return f16 ? launch_prefill_t<128, _Float16>(p, stream)
               : launch_prefill_t<128, float>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace mi
