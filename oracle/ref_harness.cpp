// ref_harness.cpp -- drives the reference engine's own attention ops.
//
// TEST INFRASTRUCTURE ONLY. Compiled (by oracle/Makefile) together with the
// reference's sources where they lie, into oracle/_ref/libmi_ref.so, which
// never enters the repository's history. It builds the three attention nodes
// with the reference's own builders (src/graph.cpp:156-163, 241-253, 263-273)
// over caller-owned buffers and runs them with the reference's own executor
// (src/graph.cpp:75-83 -> src/threadpool.cpp:237-251), so its outputs are the
// reference's outputs bit for bit. Used to write the golden vectors in
// tests/golden/ and, where present, as the timed CPU baseline.
#include <algorithm>
#include <chrono>
#include <cstddef>
#include <cstdint>
#include <vector>

#include "context.h"
#include "graph.h"
#include "ops_cpu.h"
#include "quant.h"
#include "threadpool.h"

namespace {

struct Built {
  mi_context* ctx = nullptr;
  mi_cgraph* graph = nullptr;
};

// One or more layers' attention triples in one graph, each layer's nodes
// built from its own q/k/v/out buffers, scores/probs buffers shared (they are
// dead after each layer's ATTN_KQV, as the engine's allocator would reuse).
Built build(const float* const* q, const float* const* k, const float* const* v, float* scores,
            float* probs, float* const* out, int n_layers, int head_dim, int n_head,
            int n_head_kv, int n_ctx, int n_past, int n_tokens, float scale) {
  Built b;
  mi_context_params cp{};
  cp.tensor_capacity = 16 + 8 * (size_t)n_layers;
  cp.data_capacity = 4096 + 64 * (size_t)n_layers * sizeof(void*) * 3;
  cp.no_alloc = true;
  b.ctx = mi_context_new(cp);
  const int n_rep = n_head / n_head_kv;
  b.graph = mi_graph_new(b.ctx, 8 + 8 * n_layers);
  for (int l = 0; l < n_layers; ++l) {
    int64_t qne[3] = {head_dim, n_head, n_tokens};
    int64_t kne[3] = {head_dim, n_head_kv, n_ctx};
    mi_tensor* tq = mi_context_new_tensor_from_data(b.ctx, MI_TYPE_F32, 3, qne, (void*)q[l]);
    mi_tensor* tk = mi_context_new_tensor_from_data(b.ctx, MI_TYPE_F32, 3, kne, (void*)k[l]);
    mi_tensor* tv = mi_context_new_tensor_from_data(b.ctx, MI_TYPE_F32, 3, kne, (void*)v[l]);
    tk->flags = MI_TENSOR_FLAG_KV;
    tv->flags = MI_TENSOR_FLAG_KV;
    mi_tensor* s = mi_graph_attn_qk(b.ctx, tq, tk, n_past, n_rep);
    s->data = scores;
    mi_tensor* p = mi_graph_softmax(b.ctx, s, n_past, scale);
    p->data = probs;
    mi_tensor* o = mi_graph_attn_kqv(b.ctx, p, tv, n_rep);
    o->data = out[l];
    if (l == 0)
      mi_graph_build_forward(b.graph, o);
    else
      mi_graph_build_forward_expand(b.graph, o);
  }
  return b;
}

}  // namespace

extern "C" {

// Reference ATTN_QK -> SOFTMAX -> ATTN_KQV on contiguous buffers (same
// argument meaning as oracle_attention in attn_oracle.cpp). 0 on success.
int ref_attention(const float* q, const float* k, const float* v, float* scores, float* probs,
                  float* out, int head_dim, int n_head, int n_head_kv, int n_ctx, int n_past,
                  int n_tokens, float scale, int n_threads) {
  if (head_dim <= 0 || n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv != 0 || n_past < 0 ||
      n_tokens <= 0 || n_past + n_tokens > n_ctx)
    return -1;
  Built b = build(&q, &k, &v, scores, probs, &out, 1, head_dim, n_head, n_head_kv, n_ctx, n_past,
                  n_tokens, scale);
  mi_threadpool_params tp{n_threads > 0 ? n_threads : 1, false, MI_MULMAT_STATIC, 8};
  mi_threadpool* pool = mi_threadpool_new(tp);
  mi_graph_compute(b.graph, pool);
  mi_threadpool_free(pool);
  mi_context_free(b.ctx);
  return 0;
}

// Reference MI_OP_SOFTMAX alone on a contiguous [n_kv, n_tokens, n_head] input.
int ref_softmax(const float* src, float* dst, int n_kv, int n_tokens, int n_head, int n_past,
                float scale) {
  mi_context_params cp{};
  cp.tensor_capacity = 4;
  cp.data_capacity = 0;
  cp.no_alloc = true;
  mi_context* ctx = mi_context_new(cp);
  int64_t ne[3] = {n_kv, n_tokens, n_head};
  mi_tensor* s = mi_context_new_tensor_from_data(ctx, MI_TYPE_F32, 3, ne, (void*)src);
  mi_tensor* p = mi_graph_softmax(ctx, s, n_past, scale);
  p->data = dst;
  mi_compute_softmax(p, 0, 1);
  mi_context_free(ctx);
  return 0;
}

// Reference MI_OP_ROPE (src/graph.cpp:146-154 builder, src/ops_cpu.cpp:270-302
// kernel) on a contiguous [head_dim, n_head, n_tokens] input, one thread.
int ref_rope(const float* src, float* dst, int head_dim, int n_head, int n_tokens, int n_past,
             int n_dims, float freq_base) {
  mi_context_params cp{};
  cp.tensor_capacity = 4;
  cp.data_capacity = 0;
  cp.no_alloc = true;
  mi_context* ctx = mi_context_new(cp);
  int64_t ne[3] = {head_dim, n_head, n_tokens};
  mi_tensor* s = mi_context_new_tensor_from_data(ctx, MI_TYPE_F32, 3, ne, (void*)src);
  mi_tensor* r = mi_graph_rope(ctx, s, n_past, n_dims, freq_base);
  r->data = dst;
  mi_compute_rope(r, 0, 1);
  mi_context_free(ctx);
  return 0;
}

float ref_fp16_to_fp32(uint16_t h) { return mi_fp16_to_fp32(h); }

// The reference's Q8_0 routines on contiguous buffers: weight rows from
// floats (src/quant.cpp:129-153), activation rows (src/quant.cpp:188-210), and
// the dot product mul_mat calls (src/quant.cpp:240-247, its runtime dispatch
// included) for every (row i, column j): dst[j * n + i].
void ref_quantize_rows_q8_0(const float* x, void* w, int64_t k, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    mi_quantize_row_q8_0(x + i * k, static_cast<block_q8_0*>(w) + i * (k / MI_QK8_0), k);
}

void ref_quantize_rows_q8_0_act(const float* x, void* act, int64_t k, int64_t m) {
  for (int64_t j = 0; j < m; ++j)
    mi_quantize_row_q8_0_act(x + j * k, static_cast<block_q8_0_act*>(act) + j * (k / MI_QK8_0), k);
}

void ref_mul_mat_q8_0(const void* w, const void* act, float* dst, int64_t k, int64_t n, int64_t m) {
  for (int64_t j = 0; j < m; ++j)
    for (int64_t i = 0; i < n; ++i)
      dst[j * n + i] = mi_vec_dot_q8_0_wact(static_cast<const block_q8_0*>(w) + i * (k / MI_QK8_0),
                                            static_cast<const block_q8_0_act*>(act) + j * (k / MI_QK8_0), k);
}

// The reference's own struct layout (src/tensor.h:122-160, src/graph.h:19-47),
// in the order of mi_hip_abi_layout.
int ref_abi_layout(size_t* out, int n) {
  if (n < 15) return -1;
  out[0] = sizeof(mi_tensor);
  out[1] = offsetof(mi_tensor, type);
  out[2] = offsetof(mi_tensor, ne);
  out[3] = offsetof(mi_tensor, nb);
  out[4] = offsetof(mi_tensor, op);
  out[5] = offsetof(mi_tensor, op_params);
  out[6] = offsetof(mi_tensor, src);
  out[7] = offsetof(mi_tensor, data);
  out[8] = offsetof(mi_tensor, view_src);
  out[9] = offsetof(mi_tensor, view_offs);
  out[10] = offsetof(mi_tensor, n_children);
  out[11] = offsetof(mi_tensor, flags);
  out[12] = offsetof(mi_tensor, name);
  out[13] = offsetof(mi_tensor, extra);
  out[14] = sizeof(mi_cgraph);
  return 0;
}

void ref_fp16_to_fp32_row(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = mi_fp16_to_fp32(src[i]);
}

// Median seconds of `reps` executions of n_layers attention triples (one
// graph, the reference's threadpool, barrier per node) after `warmup` runs.
double ref_time_attention(const float* const* q, const float* const* k, const float* const* v,
                          float* scores, float* probs, float* const* out, int n_layers,
                          int head_dim, int n_head, int n_head_kv, int n_ctx, int n_past,
                          int n_tokens, float scale, int n_threads, int warmup, int reps) {
  if (n_layers < 1 || reps < 1 || n_head % n_head_kv != 0 || n_past + n_tokens > n_ctx)
    return -1.0;
  Built b = build(q, k, v, scores, probs, out, n_layers, head_dim, n_head, n_head_kv, n_ctx,
                  n_past, n_tokens, scale);
  mi_threadpool_params tp{n_threads > 0 ? n_threads : 1, false, MI_MULMAT_STATIC, 8};
  mi_threadpool* pool = mi_threadpool_new(tp);
  for (int i = 0; i < warmup; ++i) mi_graph_compute(b.graph, pool);
  std::vector<double> t;
  for (int r = 0; r < reps; ++r) {
    auto t0 = std::chrono::steady_clock::now();
    mi_graph_compute(b.graph, pool);
    auto t1 = std::chrono::steady_clock::now();
    t.push_back(std::chrono::duration<double>(t1 - t0).count());
  }
  mi_threadpool_free(pool);
  mi_context_free(b.ctx);
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

}  // extern "C"
