// kernels.h -- host-side launchers of the HIP kernels (internal to the
// library; the public surface is include/mi_hip_attn.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "attn_common.h"

namespace mi {

// decode.hip
int decode_group_size(int n_rep);                       // G: Q heads per group
int decode_wg_waves(int head_dim, bool f16);            // waves per decode workgroup
size_t decode_record_floats(int head_dim, int group);   // floats per cross-workgroup record
int decode_team(int head_dim, bool f16, int group);     // workgroups per combine team
// p.rec / p.cnt: one record per workgroup and p.cst arrival counters per group
// (zero on entry, left zero on exit).
hipError_t launch_decode(const DecodeParams& p, int head_dim, bool f16, int group,
                         hipStream_t stream);

// prefill.hip
hipError_t launch_prefill(const PrefillParams& p, int head_dim, bool f16, int n_cu,
                          hipStream_t stream);

// nodes.hip -- node-level kernels on device tensors (byte strides).
struct NodeView {
  char* data;
  int64_t ne[3];
  int64_t nb[3];
};
hipError_t launch_attn_qk_node(const NodeView& dst, const NodeView& q, const NodeView& k,
                               bool k_f16, int n_rep, hipStream_t stream);
hipError_t launch_softmax_node(const NodeView& dst, const NodeView& src, int n_past, float scale,
                               hipStream_t stream);
hipError_t launch_attn_kqv_node(const NodeView& dst, const NodeView& probs, const NodeView& v,
                                bool v_f16, int n_rep, hipStream_t stream);

// rope.hip. freq[p] = base^(-2p / n_dims) as the host's powf computes it.
constexpr int kRopeMaxPairs = 128;  // n_dims <= 256
struct RopeNode {
  const char* src;
  char* dst;
  int64_t src_nb[3], dst_nb[3];
  int64_t rows;  // n_heads * n_tokens
  int32_t n_heads, head_dim, n_past, n_dims;
  float freq[kRopeMaxPairs];
};
struct RopeAppend {
  const char* q;  // may be null
  char* q_out;
  const char* k;
  const char* v;
  char* k_cache;  // the layer's K and V tensors (position stride c_s2, head stride c_s1)
  char* v_cache;
  int64_t q_nb[3], qo_nb[3], k_nb[3], v_nb[3];
  int64_t c_s1, c_s2;
  int32_t n_tokens, n_head, n_head_kv, head_dim, n_past, n_dims;
  float freq[kRopeMaxPairs];
};
hipError_t launch_rope_node(const RopeNode& p, hipStream_t stream);
hipError_t launch_rope_append(const RopeAppend& p, bool f16, hipStream_t stream);

// mul_mat.hip. Activation rows (F32, ne0 a multiple of 32, contiguous within
// a row) -> Q8_0_ACT blocks; Q8_0 weight rows . activation columns -> F32.
struct Q8Quantize {
  const char* src;
  char* dst;
  int64_t src_nb[4], dst_nb[4];
  int64_t ne0, ne1, ne2, rows;  // rows = ne1 * ne2 * ne3
};
struct Q8MulMat {
  const char* w;  // n rows of k/32 34-byte blocks, row i at w_nb1 * i
  const char* a;  // m columns of k/32 36-byte blocks, column j at a_nb1 * j
  char* dst;      // dst(i, j) at dst_nb0 * i + dst_nb1 * j
  int64_t w_nb1, a_nb1, dst_nb0, dst_nb1;
  int64_t k, n, m;
};
hipError_t launch_quantize_q8_0_act(const Q8Quantize& p, hipStream_t stream);
hipError_t launch_mul_mat_q8_0(const Q8MulMat& p, int n_cu, hipStream_t stream);

// Cache append: src F32 [head_dim, n_head_kv, n_tokens] (device, byte strides)
// into dst rows [pos0, pos0 + n_tokens) of a [head_dim, n_head_kv, n_ctx]
// cache with byte strides dst_s1 (head) and dst_s2 (position).
hipError_t launch_kv_append(char* dst, int64_t dst_s1, int64_t dst_s2, bool dst_f16,
                            const char* src, const int64_t src_nb[3], int head_dim,
                            int n_head_kv, int pos0, int n_tokens, hipStream_t stream);

}  // namespace mi
