// attn_oracle.cpp -- CPU restatement of the engine's attention graph ops.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP kernels are
// compared against, and the CPU baseline that bench.py times beside them. No
// product code path may call it; the HIP library never links it.
//
// It restates, in code of its own, the exact loop nest, summation order and
// float arithmetic of the reference's CPU kernels, so that its results are
// bit-identical to them (pinned by the golden vectors in tests/golden/, which
// come from the reference compiled in place, see oracle/Makefile):
//   addressing          src/ops_cpu.cpp:38-41   (byte strides nb[])
//   static thread split src/ops_cpu.cpp:46-53   (even, remainder to the front)
//   MI_OP_SOFTMAX       src/ops_cpu.cpp:304-346
//   MI_OP_ATTN_QK       src/ops_cpu.cpp:356-380
//   MI_OP_ATTN_KQV      src/ops_cpu.cpp:386-410
//   MI_OP_ROPE          src/ops_cpu.cpp:270-302 (NEOX halves; op_params of
//                       src/graph.cpp:146-154)
//   MI_OP_QUANTIZE_Q8_0 src/ops_cpu.cpp:462-479 with src/quant.cpp:188-210
//   MI_OP_MUL_MAT, Q8_0 weights: src/ops_cpu.cpp:226-236 with the dot product
//                       the reference dispatches to on AVX2 hosts
//                       (src/quant.cpp:240-247 -> src/quant_avx2.cpp:174-185,
//                       block dot :97-105, horizontal sum :74-83)
//   F16 -> F32          src/quant.cpp:26-63 (IEEE binary16 widening)
// Build flags: -O3 -ffp-contract=off, no -ffast-math, no -march: the same
// scalar float semantics as the reference's baseline x86-64 build.
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <algorithm>
#include <thread>
#include <vector>

#include "mi_tensor.h"

namespace {

// Element address from byte strides (src/ops_cpu.cpp:38-41).
inline float& elem(const mi_tensor* t, int64_t i0, int64_t i1, int64_t i2) {
  char* base = static_cast<char*>(t->data);
  return *reinterpret_cast<float*>(base + i0 * (int64_t)t->nb[0] + i1 * (int64_t)t->nb[1] +
                                   i2 * (int64_t)t->nb[2]);
}

// [lo, hi) of `n` units owned by thread `ith` of `nth`: equal shares, the
// first n % nth threads take one extra (src/ops_cpu.cpp:46-53).
inline void share_of(int64_t n, int ith, int nth, int64_t* lo, int64_t* hi) {
  const int64_t base = n / nth;
  const int64_t extra = n % nth;
  const int64_t start = ith * base + std::min<int64_t>(ith, extra);
  *lo = start;
  *hi = start + base + (ith < extra ? 1 : 0);
}

// Scores: for each (head h, key i) unit, every query column j gets
// sum_d K[d, h/n_rep, i] * Q[d, h, j], d ascending, one float accumulator,
// K operand on the left (src/ops_cpu.cpp:356-380).
void attn_qk(mi_tensor* dst, int ith, int nth) {
  const mi_tensor* q = dst->src[0];
  const mi_tensor* k = dst->src[1];
  const int64_t n_rep = mi_tensor_param_i32(dst, 1);
  const int64_t dim = q->ne[0];
  const int64_t n_head = q->ne[1];
  const int64_t n_tok = q->ne[2];
  const int64_t n_key = dst->ne[0];
  int64_t lo, hi;
  share_of(n_head * n_key, ith, nth, &lo, &hi);
  for (int64_t unit = lo; unit < hi; ++unit) {
    const int64_t h = unit / n_key;
    const int64_t key = unit % n_key;
    const int64_t g = h / n_rep;
    for (int64_t j = 0; j < n_tok; ++j) {
      float acc = 0.0f;
      for (int64_t d = 0; d < dim; ++d) acc += elem(k, d, g, key) * elem(q, d, h, j);
      elem(dst, key, j, h) = acc;
    }
  }
}

// Causal scaled softmax over keys, one row per (query j, head h); query j may
// see keys [0, n_past + j] (clamped to the row length); three passes (max,
// exp + sum, normalise by one reciprocal), masked tail written as 0
// (src/ops_cpu.cpp:304-346).
void softmax(mi_tensor* dst, int ith, int nth) {
  const mi_tensor* s = dst->src[0];
  const int64_t n_past = mi_tensor_param_i32(dst, 0);
  const float scale = mi_tensor_param_f32(dst, 1);
  const int64_t n_key = s->ne[0];
  const int64_t n_tok = s->ne[1];
  const int64_t n_head = s->ne[2];
  int64_t lo, hi;
  share_of(n_tok * n_head, ith, nth, &lo, &hi);
  for (int64_t row = lo; row < hi; ++row) {
    const int64_t j = row % n_tok;
    const int64_t h = row / n_tok;
    const int64_t visible = std::min(n_past + j + 1, n_key);
    float top = -INFINITY;
    for (int64_t i = 0; i < visible; ++i) {
      const float x = elem(s, i, j, h) * scale;
      if (x > top) top = x;
    }
    float total = 0.0f;
    for (int64_t i = 0; i < visible; ++i) {
      const float e = std::exp(elem(s, i, j, h) * scale - top);
      elem(dst, i, j, h) = e;
      total += e;
    }
    const float inv = 1.0f / total;
    for (int64_t i = 0; i < visible; ++i) elem(dst, i, j, h) *= inv;
    for (int64_t i = visible; i < n_key; ++i) elem(dst, i, j, h) = 0.0f;
  }
}

// Output: for each (head h, dim o) unit, every query column j gets
// sum_t V[o, h/n_rep, t] * P[t, j, h] over ALL keys t ascending (masked keys
// contribute exact zeros), V operand on the left (src/ops_cpu.cpp:386-410).
void attn_kqv(mi_tensor* dst, int ith, int nth) {
  const mi_tensor* p = dst->src[0];
  const mi_tensor* v = dst->src[1];
  const int64_t n_rep = mi_tensor_param_i32(dst, 0);
  const int64_t n_key = p->ne[0];
  const int64_t n_tok = p->ne[1];
  const int64_t n_head = p->ne[2];
  const int64_t dim = dst->ne[0];
  int64_t lo, hi;
  share_of(n_head * dim, ith, nth, &lo, &hi);
  for (int64_t unit = lo; unit < hi; ++unit) {
    const int64_t h = unit / dim;
    const int64_t o = unit % dim;
    const int64_t g = h / n_rep;
    for (int64_t j = 0; j < n_tok; ++j) {
      float acc = 0.0f;
      for (int64_t t = 0; t < n_key; ++t) acc += elem(v, o, g, t) * elem(p, t, j, h);
      elem(dst, o, h, j) = acc;
    }
  }
}

// Rotary position embedding, NEOX form: for each row (head i1, token i2) at
// position n_past + i2 and each p < n_dims / 2, the pair (p, p + n_dims / 2)
// is rotated by theta = pos * base^(-2p / n_dims), all in float: the
// frequency from powf, the angle one float product, cosf/sinf, and the
// rotation as two rounded products and one rounded sum or difference.
// Elements from n_dims on are copied. Rows split over threads like every
// other node (src/ops_cpu.cpp:270-302).
void rope(mi_tensor* dst, int ith, int nth) {
  const mi_tensor* src = dst->src[0];
  int32_t n_past, n_dims;
  float base;
  std::memcpy(&n_past, &dst->op_params[0], 4);
  std::memcpy(&n_dims, &dst->op_params[1], 4);
  std::memcpy(&base, &dst->op_params[2], 4);
  const int64_t head_dim = src->ne[0], n_heads = src->ne[1];
  const int64_t half = n_dims / 2;
  int64_t lo, hi;
  share_of(n_heads * src->ne[2], ith, nth, &lo, &hi);
  for (int64_t r = lo; r < hi; ++r) {
    const int64_t i1 = r % n_heads, i2 = r / n_heads;
    const int64_t pos = n_past + i2;
    for (int64_t p = 0; p < half; ++p) {
      const float freq = powf(base, -(float)(2 * p) / (float)n_dims);
      const float theta = (float)pos * freq;
      const float c = cosf(theta), sn = sinf(theta);
      const float x0 = elem(src, p, i1, i2), x1 = elem(src, p + half, i1, i2);
      elem(dst, p, i1, i2) = x0 * c - x1 * sn;
      elem(dst, p + half, i1, i2) = x0 * sn + x1 * c;
    }
    for (int64_t i = n_dims; i < head_dim; ++i) elem(dst, i, i1, i2) = elem(src, i, i1, i2);
  }
}

void set_contiguous(mi_tensor* t, int64_t ne0, int64_t ne1, int64_t ne2, void* data) {
  std::memset(t, 0, sizeof(*t));
  t->type = MI_TYPE_F32;
  t->ne[0] = ne0;
  t->ne[1] = ne1;
  t->ne[2] = ne2;
  t->ne[3] = 1;
  t->nb[0] = sizeof(float);
  t->nb[1] = t->nb[0] * (size_t)ne0;
  t->nb[2] = t->nb[1] * (size_t)ne1;
  t->nb[3] = t->nb[2] * (size_t)ne2;
  t->data = data;
}

// Persistent worker pool with a generation barrier: every worker runs every
// node with its (ith, nth) and then waits for the others, the executor
// contract of src/threadpool.cpp:171-180. Worker 0 is the calling thread.
class Pool {
 public:
  explicit Pool(int n) : n_(n < 1 ? 1 : n) {
    for (int i = 1; i < n_; ++i) workers_.emplace_back([this, i] { loop(i); });
  }
  ~Pool() {
    stop_.store(true, std::memory_order_relaxed);
    run_.fetch_add(1, std::memory_order_release);
    for (auto& w : workers_) w.join();
  }
  // Runs nodes[0..n) in order on all threads with a barrier after each.
  void run(mi_tensor* const* nodes, int n, void (*const* fns)(mi_tensor*, int, int)) {
    nodes_ = nodes;
    fns_ = fns;
    count_ = n;
    run_.fetch_add(1, std::memory_order_release);
    work(0);
  }

 private:
  void work(int ith) {
    for (int i = 0; i < count_; ++i) {
      fns_[i](nodes_[i], ith, n_);
      barrier();
    }
  }
  void barrier() {
    const uint32_t gen = gen_.load(std::memory_order_relaxed);
    if (arrived_.fetch_add(1, std::memory_order_acq_rel) + 1 == n_) {
      arrived_.store(0, std::memory_order_relaxed);
      gen_.fetch_add(1, std::memory_order_release);
    } else {
      while (gen_.load(std::memory_order_acquire) == gen) std::this_thread::yield();
    }
  }
  void loop(int ith) {
    uint32_t seen = 0;
    for (;;) {
      uint32_t r;
      while ((r = run_.load(std::memory_order_acquire)) == seen) std::this_thread::yield();
      seen = r;
      if (stop_.load(std::memory_order_relaxed)) return;
      work(ith);
    }
  }
  int n_;
  std::vector<std::thread> workers_;
  std::atomic<uint32_t> run_{0};
  std::atomic<uint32_t> gen_{0};
  std::atomic<int> arrived_{0};
  std::atomic<bool> stop_{false};
  mi_tensor* const* nodes_ = nullptr;
  void (*const* fns_)(mi_tensor*, int, int) = nullptr;
  int count_ = 0;
};

struct Problem {
  mi_tensor q, k, v, scores, probs, out;
  mi_tensor* nodes[3];
};

// Wires the three nodes exactly as src/model_qwen2.cpp:169-172 does through
// the builders of src/graph.cpp:156-163, 241-253, 263-273: ATTN_QK
// (op_params n_past, n_rep) -> SOFTMAX (n_past, scale) -> ATTN_KQV (n_rep).
void build(Problem* p, const float* q, const float* k, const float* v, float* scores,
           float* probs, float* out, int head_dim, int n_head, int n_head_kv, int n_ctx,
           int n_past, int n_tokens, float scale) {
  const int n_rep = n_head / n_head_kv;
  const int n_key = n_past + n_tokens;
  set_contiguous(&p->q, head_dim, n_head, n_tokens, const_cast<float*>(q));
  set_contiguous(&p->k, head_dim, n_head_kv, n_ctx, const_cast<float*>(k));
  set_contiguous(&p->v, head_dim, n_head_kv, n_ctx, const_cast<float*>(v));
  set_contiguous(&p->scores, n_key, n_tokens, n_head, scores);
  p->scores.op = MI_OP_ATTN_QK;
  p->scores.src[0] = &p->q;
  p->scores.src[1] = &p->k;
  p->scores.op_params[0] = n_past;
  p->scores.op_params[1] = n_rep;
  set_contiguous(&p->probs, n_key, n_tokens, n_head, probs);
  p->probs.op = MI_OP_SOFTMAX;
  p->probs.src[0] = &p->scores;
  p->probs.op_params[0] = n_past;
  std::memcpy(&p->probs.op_params[1], &scale, sizeof(float));
  set_contiguous(&p->out, head_dim, n_head, n_tokens, out);
  p->out.op = MI_OP_ATTN_KQV;
  p->out.src[0] = &p->probs;
  p->out.src[1] = &p->v;
  p->out.op_params[0] = n_rep;
  p->nodes[0] = &p->scores;
  p->nodes[1] = &p->probs;
  p->nodes[2] = &p->out;
}

void (*const kFns[3])(mi_tensor*, int, int) = {attn_qk, softmax, attn_kqv};

bool valid(int head_dim, int n_head, int n_head_kv, int n_ctx, int n_past, int n_tokens) {
  return head_dim > 0 && n_head > 0 && n_head_kv > 0 && n_head % n_head_kv == 0 &&
         n_past >= 0 && n_tokens > 0 && n_past + n_tokens <= n_ctx;
}

}  // namespace

extern "C" {

void oracle_split_range(int64_t n, int ith, int nth, int64_t* lo, int64_t* hi) {
  share_of(n, ith, nth, lo, hi);
}

void oracle_attn_qk(mi_tensor* dst, int ith, int nth) { attn_qk(dst, ith, nth); }
void oracle_softmax(mi_tensor* dst, int ith, int nth) { softmax(dst, ith, nth); }
void oracle_attn_kqv(mi_tensor* dst, int ith, int nth) { attn_kqv(dst, ith, nth); }
void oracle_rope_node(mi_tensor* dst, int ith, int nth) { rope(dst, ith, nth); }

// MI_OP_ROPE on contiguous [head_dim, n_head, n_tokens] buffers, one thread.
void oracle_rope(const float* src, float* dst, int head_dim, int n_head, int n_tokens, int n_past,
                 int n_dims, float freq_base) {
  mi_tensor s, d;
  set_contiguous(&s, head_dim, n_head, n_tokens, const_cast<float*>(src));
  set_contiguous(&d, head_dim, n_head, n_tokens, dst);
  d.op = MI_OP_ROPE;
  d.src[0] = &s;
  std::memcpy(&d.op_params[0], &n_past, 4);
  std::memcpy(&d.op_params[1], &n_dims, 4);
  std::memcpy(&d.op_params[2], &freq_base, 4);
  rope(&d, 0, 1);
}

// IEEE binary16 -> binary32, exact for every input (src/quant.cpp:26-63):
// zero, subnormal (renormalised), normal, inf and nan payloads.
float oracle_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t e = (h >> 10) & 0x1f;
  uint32_t m = h & 0x3ff;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13);
  } else if (e != 0) {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  } else if (m == 0) {
    bits = sign;
  } else {
    // value = m * 2^-24; shift the leading one up to bit 10.
    const int lead = 31 - __builtin_clz(m);  // 0..9
    const int shift = 10 - lead;
    m = (m << shift) & 0x3ff;
    bits = sign | ((uint32_t)(113 - shift) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, sizeof f);
  return f;
}

void oracle_fp16_to_fp32_row(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_fp16_to_fp32(src[i]);
}

// ---- Q8_0 ------------------------------------------------------------------
// Weight block: fp16 scale then 32 int8 (34 bytes, src/quant.h:22-28).
// Activation block: float scale then 32 int8 (36 bytes, src/quant.h:122-127).
#pragma pack(push, 1)
struct OracleBlockQ8 {
  uint16_t d;
  int8_t qs[32];
};
#pragma pack(pop)
struct OracleBlockAct {
  float d;
  int8_t qs[32];
};
static_assert(sizeof(OracleBlockQ8) == 34 && sizeof(OracleBlockAct) == 36, "Q8_0 block layouts");

// One row of n floats -> n/32 activation blocks: amax of the block (strict
// greater-than scan), d = amax / 127, id = 1 / d (0 for an all-zero block),
// q = lrintf(x * id) clamped to [-127, 127].
void oracle_quantize_row_q8_0_act(const float* x, OracleBlockAct* y, int64_t n) {
  for (int64_t i = 0; i < n / 32; ++i) {
    const float* xb = x + i * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
      const float av = std::fabs(xb[j]);
      if (av > amax) amax = av;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    y[i].d = d;
    for (int j = 0; j < 32; ++j) {
      int32_t q = (int32_t)lrintf(xb[j] * id);
      if (q > 127) q = 127;
      if (q < -127) q = -127;
      y[i].qs[j] = (int8_t)q;
    }
  }
}

// Weight row . activation row over n elements, in the order of the
// reference's default (AVX2 + FMA) dot product: eight float accumulators,
// accumulator l takes fma(float(sum of the block's int8 products 4l..4l+3),
// fp16(w.d) * a.d, acc[l]) block by block, then the horizontal sum
// ((acc0 + acc4) + (acc1 + acc5)) + ((acc2 + acc6) + (acc3 + acc7)).
float oracle_vec_dot_q8_0_act(const OracleBlockQ8* w, const OracleBlockAct* a, int64_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t i = 0; i < n / 32; ++i) {
    const float dxdy = oracle_fp16_to_fp32(w[i].d) * a[i].d;
    for (int l = 0; l < 8; ++l) {
      int32_t isum = 0;
      for (int k = 0; k < 4; ++k) isum += (int32_t)w[i].qs[4 * l + k] * (int32_t)a[i].qs[4 * l + k];
      acc[l] = std::fma((float)isum, dxdy, acc[l]);
    }
  }
  float s[4];
  for (int k = 0; k < 4; ++k) s[k] = acc[k] + acc[k + 4];
  return (s[0] + s[1]) + (s[2] + s[3]);
}

// MI_OP_MUL_MAT with Q8_0 weights a [k, n] (row i at a->nb[1] i) and a
// Q8_0_ACT activation b [k, m] (column j at b->nb[1] j): dst(i, j) =
// vec_dot(row i, column j); rows split over threads (each row's order is the
// same whichever thread computes it).
void oracle_mul_mat_q8_0(mi_tensor* dst, int ith, int nth) {
  const mi_tensor* a = dst->src[0];
  const mi_tensor* b = dst->src[1];
  const int64_t k = a->ne[0], n = a->ne[1], m = b->ne[1];
  int64_t lo, hi;
  share_of(n, ith, nth, &lo, &hi);
  for (int64_t i = lo; i < hi; ++i) {
    const auto* arow = reinterpret_cast<const OracleBlockQ8*>(static_cast<const char*>(a->data) +
                                                             i * (int64_t)a->nb[1]);
    for (int64_t j = 0; j < m; ++j) {
      const auto* brow = reinterpret_cast<const OracleBlockAct*>(
          static_cast<const char*>(b->data) + j * (int64_t)b->nb[1]);
      elem(dst, i, j, 0) = oracle_vec_dot_q8_0_act(arow, brow, k);
    }
  }
}

// Contiguous forms: x [m][k] floats -> act [m][k/32] blocks; W [n][k/32]
// blocks . act -> dst [m][n] (dst(i, j) at j * n + i, the engine's [n, m]).
void oracle_quantize_q8_0_act(const float* x, void* act, int64_t k, int64_t m) {
  for (int64_t j = 0; j < m; ++j)
    oracle_quantize_row_q8_0_act(x + j * k, static_cast<OracleBlockAct*>(act) + j * (k / 32), k);
}

void oracle_mul_mat_q8_0_contig(const void* w, const void* act, float* dst, int64_t k, int64_t n,
                                int64_t m) {
  for (int64_t j = 0; j < m; ++j)
    for (int64_t i = 0; i < n; ++i)
      dst[j * n + i] = oracle_vec_dot_q8_0_act(static_cast<const OracleBlockQ8*>(w) + i * (k / 32),
                                               static_cast<const OracleBlockAct*>(act) + j * (k / 32), k);
}

// Runs ATTN_QK -> SOFTMAX -> ATTN_KQV on contiguous buffers:
// q [head_dim, n_head, n_tokens], k/v [head_dim, n_head_kv, n_ctx],
// scores/probs [n_past+n_tokens, n_tokens, n_head], out [head_dim, n_head, n_tokens].
// Returns 0, or -1 on inconsistent sizes.
int oracle_attention(const float* q, const float* k, const float* v, float* scores, float* probs,
                     float* out, int head_dim, int n_head, int n_head_kv, int n_ctx, int n_past,
                     int n_tokens, float scale, int n_threads) {
  if (!valid(head_dim, n_head, n_head_kv, n_ctx, n_past, n_tokens)) return -1;
  Problem p;
  build(&p, q, k, v, scores, probs, out, head_dim, n_head, n_head_kv, n_ctx, n_past, n_tokens,
        scale);
  if (n_threads <= 1) {
    for (int i = 0; i < 3; ++i) kFns[i](p.nodes[i], 0, 1);
  } else {
    Pool pool(n_threads);
    pool.run(p.nodes, 3, kFns);
  }
  return 0;
}

// Median wall time (seconds) of `reps` runs of the three-node pass over
// n_layers independent layer problems laid out back to back (q/k/v/out are
// arrays of per-layer pointers), after `warmup` untimed runs, on a persistent
// pool of n_threads (the executor's barrier-per-node contract).
double oracle_time_attention(const float* const* q, const float* const* k,
                             const float* const* v, float* scores, float* probs,
                             float* const* out, int n_layers, int head_dim, int n_head,
                             int n_head_kv, int n_ctx, int n_past, int n_tokens, float scale,
                             int n_threads, int warmup, int reps) {
  if (!valid(head_dim, n_head, n_head_kv, n_ctx, n_past, n_tokens) || n_layers < 1 || reps < 1)
    return -1.0;
  std::vector<Problem> probs_(n_layers);
  std::vector<mi_tensor*> nodes;
  std::vector<void (*)(mi_tensor*, int, int)> fns;
  for (int l = 0; l < n_layers; ++l) {
    build(&probs_[l], q[l], k[l], v[l], scores, probs, out[l], head_dim, n_head, n_head_kv, n_ctx,
          n_past, n_tokens, scale);
    for (int i = 0; i < 3; ++i) {
      nodes.push_back(probs_[l].nodes[i]);
      fns.push_back(kFns[i]);
    }
  }
  Pool pool(n_threads);
  for (int i = 0; i < warmup; ++i) pool.run(nodes.data(), (int)nodes.size(), fns.data());
  std::vector<double> t;
  for (int r = 0; r < reps; ++r) {
    auto t0 = std::chrono::steady_clock::now();
    pool.run(nodes.data(), (int)nodes.size(), fns.data());
    auto t1 = std::chrono::steady_clock::now();
    t.push_back(std::chrono::duration<double>(t1 - t0).count());
  }
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

}  // extern "C"
