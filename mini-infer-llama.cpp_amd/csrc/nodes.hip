// nodes.hip -- the engine's attention graph ops one node at a time on device
// tensors, plus the KV-cache append.
//
// These are the unfused counterparts of the decode/prefill kernels: they
// materialise scores and probabilities exactly like the CPU graph does, so a
// caller can run any single ATTN_QK, SOFTMAX or ATTN_KQV node on the GPU.
// ATTN_QK and ATTN_KQV accumulate with separately rounded multiply and add
// (floating-point contraction is switched off in their bodies, so no fused
// multiply-add is formed) in the reference's order --
// d ascending for scores, t ascending over all keys for the output -- so on
// identical inputs they reproduce src/ops_cpu.cpp:356-380 and :386-410 bit
// for bit. SOFTMAX reproduces src/ops_cpu.cpp:304-346 bit for bit too: the
// glibc expf restated (libm_ref.h), the running sum as one rounded add per key
// in key order, and the correctly rounded 1.0f / sum.
#include "attn_common.h"
#include "kernels.h"
#define MI_LIBM_HD __host__ __device__
#include "libm_ref.h"

namespace mi {

static __constant__ uint64_t kExpfTab[32] = MI_EXPF_TABLE;

template <typename T>
__device__ inline float ld(const NodeView& t, int64_t i0, int64_t i1, int64_t i2) {
  return (float)*reinterpret_cast<const T*>(t.data + i0 * t.nb[0] + i1 * t.nb[1] + i2 * t.nb[2]);
}

__device__ inline float& at(const NodeView& t, int64_t i0, int64_t i1, int64_t i2) {
  return *reinterpret_cast<float*>(t.data + i0 * t.nb[0] + i1 * t.nb[1] + i2 * t.nb[2]);
}

// dst [n_kv, n_tokens, n_head]: S[i,j,h] = sum_d K[d, h/n_rep, i] * Q[d, h, j].
template <typename KT>
__global__ void attn_qk_node_kernel(NodeView dst, NodeView q, NodeView k, int n_rep) {
#pragma clang fp contract(off)
  const int64_t n_kv = dst.ne[0], n_tok = dst.ne[1], n_head = dst.ne[2], dim = q.ne[0];
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n_kv * n_tok * n_head) return;
  const int64_t i = idx % n_kv;
  const int64_t j = (idx / n_kv) % n_tok;
  const int64_t h = idx / (n_kv * n_tok);
  const int64_t g = h / n_rep;
  float acc = 0.f;
  for (int64_t d = 0; d < dim; ++d) acc = acc + ld<KT>(k, d, g, i) * ld<float>(q, d, h, j);
  at(dst, i, j, h) = acc;
}

// One wave per (token j, head h) row: causal scaled softmax over keys
// [0, min(n_past + j + 1, n_kv)), zeros beyond. The maximum is order-free;
// the sum follows the reference's order: per chunk of 64 keys every lane
// computes and stores its e, then the wave adds the chunk's values one at a
// time, lane k's k-th (a uniform running sum).
__global__ void softmax_node_kernel(NodeView dst, NodeView src, int n_past, float scale) {
#pragma clang fp contract(off)
  const int64_t n_kv = src.ne[0], n_tok = src.ne[1];
  const int64_t row = blockIdx.x;
  const int64_t j = row % n_tok, h = row / n_tok;
  const int64_t visible = min((int64_t)n_past + j + 1, n_kv);
  const int lane = threadIdx.x;
  float mx = -INFINITY;
  for (int64_t i = lane; i < visible; i += kWave) {
    const float v = ld<float>(src, i, j, h) * scale;
    mx = v > mx ? v : mx;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off);
    mx = o > mx ? o : mx;
  }
  float sum = 0.f;
  for (int64_t c = 0; c < visible; c += kWave) {
    const int64_t i = c + lane;
    float e = 0.f;
    if (i < visible) {
      e = expf_ref(ld<float>(src, i, j, h) * scale - mx, kExpfTab);
      at(dst, i, j, h) = e;
    }
    const int n = (int)min<int64_t>(kWave, visible - c);
    const int eb = __builtin_bit_cast(int, e);
    for (int k = 0; k < n; ++k) sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(eb, k));
  }
  const float inv = (float)(1.0 / (double)sum);  // the correctly rounded 1.0f / sum
  for (int64_t i = lane; i < visible; i += kWave) at(dst, i, j, h) = at(dst, i, j, h) * inv;
  for (int64_t i = visible + lane; i < n_kv; i += kWave) at(dst, i, j, h) = 0.f;
}

// dst [head_dim, n_head, n_tokens]: O[o,h,j] = sum_t V[o, h/n_rep, t] * P[t, j, h].
template <typename VT>
__global__ void attn_kqv_node_kernel(NodeView dst, NodeView probs, NodeView v, int n_rep) {
#pragma clang fp contract(off)
  const int64_t dim = dst.ne[0], n_head = dst.ne[1], n_tok = dst.ne[2], n_kv = probs.ne[0];
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= dim * n_head * n_tok) return;
  const int64_t o = idx % dim;
  const int64_t h = (idx / dim) % n_head;
  const int64_t j = idx / (dim * n_head);
  const int64_t g = h / n_rep;
  float acc = 0.f;
  for (int64_t t = 0; t < n_kv; ++t) acc = acc + ld<VT>(v, o, g, t) * ld<float>(probs, t, j, h);
  at(dst, o, h, j) = acc;
}

template <typename CT>
__global__ void kv_append_kernel(char* dst, int64_t s1, int64_t s2, const char* src, int64_t n0,
                                 int64_t n1, int64_t n2, int64_t dim, int64_t n_hkv, int pos0,
                                 int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t d = idx % dim;
  const int64_t g = (idx / dim) % n_hkv;
  const int64_t t = idx / (dim * n_hkv);
  const float x = *reinterpret_cast<const float*>(src + d * n0 + g * n1 + t * n2);
  *reinterpret_cast<CT*>(dst + (pos0 + t) * s2 + g * s1 + d * (int64_t)sizeof(CT)) = (CT)x;
}

static unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

hipError_t launch_attn_qk_node(const NodeView& dst, const NodeView& q, const NodeView& k,
                               bool k_f16, int n_rep, hipStream_t stream) {
  const int64_t n = dst.ne[0] * dst.ne[1] * dst.ne[2];
  if (n == 0) return hipSuccess;
  if (k_f16)
    hipLaunchKernelGGL(attn_qk_node_kernel<_Float16>, dim3(blocks_for(n, 256)), dim3(256), 0,
                       stream, dst, q, k, n_rep);
  else
    hipLaunchKernelGGL(attn_qk_node_kernel<float>, dim3(blocks_for(n, 256)), dim3(256), 0, stream,
                       dst, q, k, n_rep);
  return hipGetLastError();
}

hipError_t launch_softmax_node(const NodeView& dst, const NodeView& src, int n_past, float scale,
                               hipStream_t stream) {
  const int64_t rows = src.ne[1] * src.ne[2];
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(softmax_node_kernel, dim3((unsigned)rows), dim3(kWave), 0, stream, dst, src,
                     n_past, scale);
  return hipGetLastError();
}

hipError_t launch_attn_kqv_node(const NodeView& dst, const NodeView& probs, const NodeView& v,
                                bool v_f16, int n_rep, hipStream_t stream) {
  const int64_t n = dst.ne[0] * dst.ne[1] * dst.ne[2];
  if (n == 0) return hipSuccess;
  if (v_f16)
    hipLaunchKernelGGL(attn_kqv_node_kernel<_Float16>, dim3(blocks_for(n, 256)), dim3(256), 0,
                       stream, dst, probs, v, n_rep);
  else
    hipLaunchKernelGGL(attn_kqv_node_kernel<float>, dim3(blocks_for(n, 256)), dim3(256), 0, stream,
                       dst, probs, v, n_rep);
  return hipGetLastError();
}

hipError_t launch_kv_append(char* dst, int64_t dst_s1, int64_t dst_s2, bool dst_f16,
                            const char* src, const int64_t src_nb[3], int head_dim,
                            int n_head_kv, int pos0, int n_tokens, hipStream_t stream) {
  const int64_t total = (int64_t)head_dim * n_head_kv * n_tokens;
  if (total == 0) return hipSuccess;
  if (dst_f16)
    hipLaunchKernelGGL(kv_append_kernel<_Float16>, dim3(blocks_for(total, 256)), dim3(256), 0,
                       stream, dst, dst_s1, dst_s2, src, src_nb[0], src_nb[1], src_nb[2],
                       (int64_t)head_dim, (int64_t)n_head_kv, pos0, total);
  else
    hipLaunchKernelGGL(kv_append_kernel<float>, dim3(blocks_for(total, 256)), dim3(256), 0, stream,
                       dst, dst_s1, dst_s2, src, src_nb[0], src_nb[1], src_nb[2],
                       (int64_t)head_dim, (int64_t)n_head_kv, pos0, total);
  return hipGetLastError();
}

}  // namespace mi
