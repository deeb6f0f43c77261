// kernels.h -- host-side launchers of the HIP kernels (internal to the
// library; the public surface is include/mi_hip_attn.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "attn_common.h"

namespace mi {

// decode.hip
int decode_chunks(int n_rep);                           // head chunks per KV head
int decode_group_size(int n_rep);                       // G: Q heads of the widest chunk
int decode_wg_waves(int head_dim, bool f16);            // waves per decode workgroup
int decode_ring_slots(int head_dim, bool f16);          // ring slots per wave
size_t decode_record_floats(int head_dim, int group);   // floats per cross-workgroup record
int decode_team(int head_dim, bool f16, int group);     // workgroups per combine team
// p.rec: one record per workgroup; p.cnt: two counter sets (the set of the
// launch's epoch parity is zero on entry; the other is cleared). By default
// every workgroup, kpg > 1 included, takes fixed strided sub-tiles of its
// group (part p: p, p + kpg, ...) through an LDS counter; dyn (opt-in,
// MI_HIP_DECODE_CLAIM) has the waves claim sub-tiles from the group's
// counter in device memory instead.
// Grid (grid_x, n_items): row y serves p.item[y]; workgroups past an item's
// gpi * kpg leave at once.
hipError_t launch_decode(const DecodeParams& p, int grid_x, int n_items, int head_dim, bool f16, int group,
                         bool dyn, bool mf, hipStream_t stream);
// decode_stream.hip: the streaming decode kernel for launches whose groups
// span several workgroups (float products, K/V straight into registers, the
// merge by the last part to arrive). head_dim 64 or 128, F32 or F16 cache,
// group <= 8 heads; p.rec_words >= stream_record_words(head_dim, group).
size_t stream_record_words(int head_dim, int group);
hipError_t launch_stream_decode(const DecodeParams& p, int grid_x, int n_items, int head_dim, bool f16, int group,
                                hipStream_t stream);
// n words at p set to v on `stream` (a kernel, so it may sit in a graph).
hipError_t launch_fill_u32(unsigned* p, size_t n, unsigned v, hipStream_t stream);

// prefill.hip. split: the QK and PV products on the bf16 matrix cores with
// operands split into hi + lo bf16 pairs (three products each); otherwise
// v_mfma_f32_32x32x2f32.
hipError_t launch_prefill(const PrefillParams& p, int head_dim, bool f16, int n_cu, bool split,
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
  // Optional table of (cos, sin) pairs, float2 at [pos * n_dims / 2 + p],
  // covering every position the launch touches: the angles' cosine and sine
  // as the host's libm returns them (the engine's own values), replacing the
  // device's correctly rounded ones.
  const float* cs = nullptr;
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
// RoPE and the K/V append as the epilogue of the stacked Q/K/V projection
// (one column): rows are n_q Q rows then n_kv K rows then n_kv V rows, Q and K
// rows permuted within each head of hd rows so that row 2j holds dim j and row
// 2j + 1 dim j + hd/2 (a rotation pair in one 8-row group). Q lands roped in
// natural order at q_out, K roped and V as is in the cache rows of position
// pos (element (head h, dim d) at k_row / v_row + h * c_s1 + 4 d).
struct RopeEpi {
  const float* cs;  // (cos, sin) pairs, float2 at [pos * hd/2 + j]
  float* q_out;
  char* k_row;
  char* v_row;
  int64_t c_s1;
  int32_t pos, hd, n_q, n_kv;
};

struct Q8MulMat {
  const char* w;  // n rows of k/32 34-byte blocks, row i at w_nb1 * i
  const char* a;  // m columns of k/32 36-byte blocks, column j at a_nb1 * j
  char* dst;      // dst(i, j) at dst_nb0 * i + dst_nb1 * j
  int64_t w_nb1, a_nb1, dst_nb0, dst_nb1;
  int64_t k, n, m;
  // Optional F32 term added to each product after it is complete (a bias with
  // add_nb1 = 0, or a residual; it may alias dst): dst(i, j) = dot + add(i, j),
  // the engine's separate ADD node (src/ops_cpu.cpp:172-175) fused.
  const char* add = nullptr;
  int64_t add_nb0 = 0, add_nb1 = 0;
  // Optional activation prologue (streaming form only, q8_ring_form): instead
  // of Q8_0_ACT blocks at `a`, each workgroup quantises the m F32 columns at x
  // (x_ld floats apart) itself, after RMS_NORM * norm_w when norm_w is set
  // (src/ops_cpu.cpp:143-170) -- the separate norm / quantize launches fused.
  const float* x = nullptr;
  int64_t x_ld = 0;
  const float* norm_w = nullptr;
  float eps = 0.0f;
  // Optional SwiGLU epilogue (streaming form, one column, q8_swiglu_out_ok):
  // the rows are gate/up pairs (row 2i is gate_i, row 2i + 1 is up_i), and
  // instead of F32 rows the kernel writes SiLU(gate_i) * up_i as Q8_0_ACT
  // blocks (block j, elements 32 j .. 32 j + 31, at swiglu_out + 36 j) -- the
  // engine's SILU, MUL and QUANTIZE nodes after the FFN gate/up projections
  // (src/model_qwen2.cpp:188-189, src/ops_cpu.cpp:412) fused.
  char* swiglu_out = nullptr;
  // Rows of the first perm_rows permuted within heads of perm_hd rows as
  // RopeEpi describes; the stores put them back in natural order (0: none).
  int32_t perm_hd = 0;
  int64_t perm_rows = 0;
  // With rope_on (streaming form, m = 1): the RopeEpi stores replace dst's.
  int32_t rope_on = 0;
  RopeEpi rope{};
};

// The natural row of stored row r of a matrix whose first perm_rows rows are
// permuted within heads of hd rows (row 2j <- dim j, 2j + 1 <- dim j + hd/2).
__host__ __device__ inline int64_t q8_unperm_row(int64_t r, int32_t hd, int64_t perm_rows) {
  if (hd == 0 || r >= perm_rows) return r;
  const int64_t head = r / hd, w = r - head * hd;
  return head * hd + (w >> 1) + (w & 1) * (hd / 2);
}
// Whether launch_mul_mat_q8_0 takes the streaming form for p (the only form
// with the activation prologue).
bool q8_ring_form(const Q8MulMat& p);
// Whether launch_mul_mat_q8_0 can run p with its SwiGLU epilogue (the
// streaming form, one column, no added term or RoPE, n a multiple of 64 and
// at most one workgroup per 64 rows on the device).
bool q8_swiglu_out_ok(const Q8MulMat& p, int n_cu);
hipError_t launch_quantize_q8_0_act(const Q8Quantize& p, hipStream_t stream);
hipError_t launch_mul_mat_q8_0(const Q8MulMat& p, int n_cu, hipStream_t stream);

// Cache append: src F32 [head_dim, n_head_kv, n_tokens] (device, byte strides)
// into dst rows [pos0, pos0 + n_tokens) of a [head_dim, n_head_kv, n_ctx]
// cache with byte strides dst_s1 (head) and dst_s2 (position).
hipError_t launch_kv_append(char* dst, int64_t dst_s1, int64_t dst_s2, bool dst_f16,
                            const char* src, const int64_t src_nb[3], int head_dim,
                            int n_head_kv, int pos0, int n_tokens, hipStream_t stream);

// attn_exact.hip: the attention triple in the reference's operation order
// (F32 K/V, head_dim a multiple of 4, n_past + n_tokens <= kExactMaxKeys).
constexpr int kExactMaxKeys = 32768;
struct ExactAttn {
  const char* q;  // [head_dim, n_head, n_tokens], byte strides q_s1 (head), q_s2 (token)
  const char* k;  // cache rows: k_s1 (KV head), k_s2 (position)
  const char* v;
  char* out;      // [head_dim, n_head, n_tokens], o_s1, o_s2
  int64_t q_s1, q_s2, k_s1, k_s2, v_s1, v_s2, o_s1, o_s2;
  int32_t n_head, n_rep, n_past, n_tokens, head_dim;
  float scale;
};
hipError_t launch_attn_exact(const ExactAttn& p, hipStream_t stream);

// Host helpers of the library's entry points (runtime.hip), for the other
// host files: the thread's last-error message, the accounted device
// allocator, selecting the library's device, and its compute-unit count.
// The read-bandwidth ceiling pass (memread.hip): n_sums workgroups, one float each.
hipError_t launch_memread(const void* src, size_t bytes, float* sums, int n_sums, hipStream_t stream);

int rt_fail(int code, const char* msg);
int rt_hip_fail(hipError_t e, const char* what);
int rt_alloc(void** p, size_t bytes, const char* what);
void rt_free(void* p, size_t bytes);
int rt_bind();
int rt_n_cu();

}  // namespace mi
