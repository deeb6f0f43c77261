// rope.hip -- rotary position embedding (MI_OP_ROPE, src/ops_cpu.cpp:270-302)
// on device tensors, and its fusion with one layer's KV-cache append
// (src/model_qwen2.cpp:153-159: rope Q, rope K, copy K and V into the cache).
//
// Arithmetic, per row at position pos and pair p < n_dims / 2, as the engine:
//   theta = pos * freq[p]           (one rounded float product; freq[p] is the
//                                    host's powf(base, -(2p)/n_dims), passed in)
//   c, s  = cos(theta), sin(theta)  (computed in double and rounded to float,
//                                    so within one float ulp of the host's
//                                    cosf/sinf, which are not correctly rounded)
//   y0 = x0 c - x1 s, y1 = x0 s + x1 c  (two rounded products and one rounded
//                                    sum each; no fused multiply-add)
// Elements from n_dims on are copied. The work is tiny and HBM-bound: one
// thread per pair (or per two copied elements) of a row, rows contiguous in
// the thread index so that a wave reads whole rows.
#include <cmath>

#include "attn_common.h"
#include "kernels.h"

namespace mi {

__device__ inline void rope_angle(int pos, float freq, float& c, float& s) {
  const float theta = (float)pos * freq;
  double sd, cd;
  sincos((double)theta, &sd, &cd);
  c = (float)cd;
  s = (float)sd;
}

__device__ inline void rope_rotate(float x0, float x1, float c, float s, float& y0, float& y1) {
#pragma clang fp contract(off)
  y0 = x0 * c - x1 * s;
  y1 = x0 * s + x1 * c;
}

__device__ inline float ldf(const char* base, int64_t off) {
  return *reinterpret_cast<const float*>(base + off);
}

// Node: dst [head_dim, n_heads, n_tokens] = rope(src). Row r = (head, token),
// lane j of the row's W = half + (head_dim - n_dims) threads: j < half rotates
// pair (j, j + half), the rest copy one element each.
__global__ void rope_node_kernel(const RopeNode p) {
  const int half = p.n_dims / 2;
  const int W = half + (p.head_dim - p.n_dims);
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.rows * W) return;
  const int64_t r = idx / W;
  const int j = (int)(idx - r * W);
  const int64_t h = r % p.n_heads, t = r / p.n_heads;
  const int64_t so = h * p.src_nb[1] + t * p.src_nb[2];
  const int64_t dof = h * p.dst_nb[1] + t * p.dst_nb[2];
  if (j < half) {
    float c, s, y0, y1;
    rope_angle(p.n_past + (int)t, p.freq[j], c, s);
    rope_rotate(ldf(p.src, so + j * p.src_nb[0]), ldf(p.src, so + (j + half) * p.src_nb[0]), c, s,
                y0, y1);
    *reinterpret_cast<float*>(p.dst + dof + j * p.dst_nb[0]) = y0;
    *reinterpret_cast<float*>(p.dst + dof + (j + half) * p.dst_nb[0]) = y1;
  } else {
    const int e = p.n_dims + (j - half);
    *reinterpret_cast<float*>(p.dst + dof + e * p.dst_nb[0]) = ldf(p.src, so + e * p.src_nb[0]);
  }
}

// Fused step: rows of token t are n_head Q rows, then n_head_kv K rows, then
// n_head_kv V rows; W = head_dim / 2 threads per row. Q/K lane j < half
// rotates a pair, the others copy two tail elements; V lanes copy two
// elements. K and V land in the cache at position n_past + t.
template <typename CT>
__global__ void rope_append_kernel(const RopeAppend p) {
  const int W = p.head_dim / 2, half = p.n_dims / 2;
  const int rows_per_tok = p.n_head + 2 * p.n_head_kv;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)p.n_tokens * rows_per_tok * W) return;
  const int64_t r = idx / W;
  const int j = (int)(idx - r * W);
  const int t = (int)(r / rows_per_tok);
  int i = (int)(r - (int64_t)t * rows_per_tok);
  const int pos = p.n_past + t;
  const bool is_q = i < p.n_head;
  const bool is_k = !is_q && i < p.n_head + p.n_head_kv;
  if (is_q && !p.q) return;
  const char* src;
  const int64_t* nb;
  if (is_q) {
    src = p.q + i * p.q_nb[1] + (int64_t)t * p.q_nb[2];
    nb = p.q_nb;
  } else if (is_k) {
    i -= p.n_head;
    src = p.k + i * p.k_nb[1] + (int64_t)t * p.k_nb[2];
    nb = p.k_nb;
  } else {
    i -= p.n_head + p.n_head_kv;
    src = p.v + i * p.v_nb[1] + (int64_t)t * p.v_nb[2];
    nb = p.v_nb;
  }
  // (element, value) pairs this lane writes
  int e0, e1;
  float y0, y1;
  if (!is_q && !is_k) {
    e0 = 2 * j;
    e1 = 2 * j + 1;
    y0 = ldf(src, e0 * nb[0]);
    y1 = ldf(src, e1 * nb[0]);
  } else if (j < half) {
    e0 = j;
    e1 = j + half;
    float c, s;
    if (p.cs) {
      const float2 cs = *reinterpret_cast<const float2*>(p.cs + 2 * ((int64_t)pos * half + j));
      c = cs.x;
      s = cs.y;
    } else {
      rope_angle(pos, p.freq[j], c, s);
    }
    rope_rotate(ldf(src, e0 * nb[0]), ldf(src, e1 * nb[0]), c, s, y0, y1);
  } else {
    e0 = p.n_dims + 2 * (j - half);
    e1 = e0 + 1;
    y0 = ldf(src, e0 * nb[0]);
    y1 = ldf(src, e1 * nb[0]);
  }
  if (is_q) {
    char* o = p.q_out + i * p.qo_nb[1] + (int64_t)t * p.qo_nb[2];
    *reinterpret_cast<float*>(o + e0 * p.qo_nb[0]) = y0;
    *reinterpret_cast<float*>(o + e1 * p.qo_nb[0]) = y1;
  } else {
    char* o = (is_k ? p.k_cache : p.v_cache) + (int64_t)pos * p.c_s2 + i * p.c_s1;
    reinterpret_cast<CT*>(o)[e0] = (CT)y0;
    reinterpret_cast<CT*>(o)[e1] = (CT)y1;
  }
}

hipError_t launch_rope_node(const RopeNode& p, hipStream_t stream) {
  const int64_t n = p.rows * (p.n_dims / 2 + (p.head_dim - p.n_dims));
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rope_node_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_rope_append(const RopeAppend& p, bool f16, hipStream_t stream) {
  const int64_t n = (int64_t)p.n_tokens * (p.n_head + 2 * p.n_head_kv) * (p.head_dim / 2);
  if (n == 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (f16)
    hipLaunchKernelGGL(rope_append_kernel<_Float16>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(rope_append_kernel<float>, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mi
