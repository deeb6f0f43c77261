// attn_exact.hip -- ATTN_QK -> causal SOFTMAX -> ATTN_KQV in the reference's
// own operation order (src/ops_cpu.cpp:304-410), bit for bit:
//
//   S_i  = sum_d K[d, kvh, i] * Q[d, h, j]     d ascending, product and sum
//                                              each rounded (no fused multiply-add)
//   v_i  = S_i * scale;  m = max_i v_i         i < a = min(n_past + j + 1, n_kv)
//   e_i  = expf(v_i - m)                       the host C library's expf (libm_ref.h)
//   sum  = sum_i e_i                           i ascending
//   P_i  = e_i * (1 / sum)
//   O[o] = sum_t V[o, kvh, t] * P_t            t ascending (masked t add +-0, skipped)
//
// One wave per (token j, head h): lanes split the keys for the scores and the
// exponentials, lane 0 runs the ordered sum, and lanes split the output
// elements for the ordered V sums. The ordered sums make a row's cost linear
// in its key count on one lane: this is the checking path for whole-model
// parity (token ids equal to the reference engine's), not the throughput path
// (decode.hip / prefill.hip).
#include <cmath>

#include "attn_common.h"
#include "kernels.h"

#define MI_LIBM_HD __host__ __device__
#include "libm_ref.h"

namespace mi {

static __constant__ uint64_t kExpfTab[32] = MI_EXPF_TABLE;

__global__ __launch_bounds__(kWave) void attn_exact_kernel(const ExactAttn p) {
#pragma clang fp contract(off)
  extern __shared__ float prob[];
  __shared__ float s_inv;
  const int lane = threadIdx.x;
  const int h = blockIdx.x % p.n_head;
  const int j = blockIdx.x / p.n_head;
  const int kvh = h / p.n_rep;
  const int D = p.head_dim;
  const int a = min(p.n_past + j + 1, p.n_past + p.n_tokens);
  const float* q = reinterpret_cast<const float*>(p.q + h * p.q_s1 + (int64_t)j * p.q_s2);
  float mx = -INFINITY;
  for (int i = lane; i < a; i += kWave) {
    const float* kr = reinterpret_cast<const float*>(p.k + kvh * p.k_s1 + (int64_t)i * p.k_s2);
    float acc = 0.0f;
    for (int d = 0; d < D; d += 4) {
      const float4 kv = *reinterpret_cast<const float4*>(kr + d);
      const float4 qv = *reinterpret_cast<const float4*>(q + d);
      acc = acc + kv.x * qv.x;
      acc = acc + kv.y * qv.y;
      acc = acc + kv.z * qv.z;
      acc = acc + kv.w * qv.w;
    }
    const float v = acc * p.scale;
    prob[i] = v;
    mx = v > mx ? v : mx;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off);
    mx = o > mx ? o : mx;
  }
  for (int i = lane; i < a; i += kWave) prob[i] = expf_ref(prob[i] - mx, kExpfTab);
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (int i = 0; i < a; ++i) sum = sum + prob[i];
    s_inv = (float)(1.0 / (double)sum);  // the correctly rounded 1.0f / sum
  }
  __syncthreads();
  const float inv = s_inv;
  for (int i = lane; i < a; i += kWave) prob[i] = prob[i] * inv;
  __syncthreads();
  float* out = reinterpret_cast<float*>(p.out + h * p.o_s1 + (int64_t)j * p.o_s2);
  const char* vbase = p.v + kvh * p.v_s1;
  for (int o = lane; o < D; o += kWave) {
    float acc = 0.0f;
    for (int t = 0; t < a; ++t)
      acc = acc + *reinterpret_cast<const float*>(vbase + (int64_t)t * p.v_s2 + 4 * o) * prob[t];
    out[o] = acc;
  }
}

hipError_t launch_attn_exact(const ExactAttn& p, hipStream_t stream) {
  const int n_kv = p.n_past + p.n_tokens;
  const size_t lds = (size_t)n_kv * sizeof(float);
  static const hipError_t attr = hipFuncSetAttribute(
      (const void*)&attn_exact_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kExactMaxKeys * 4);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(attn_exact_kernel, dim3((unsigned)(p.n_tokens * p.n_head)), dim3(kWave), lds,
                     stream, p);
  return hipGetLastError();
}

}  // namespace mi
