// qwen2.hip -- a Qwen2 decoder resident on one GPU (include/mi_hip_qwen2.h):
// the reference engine's forward graph (src/model_qwen2.cpp:133-234) as a
// fixed sequence of launches on one stream, around the fused attention.
//
// Device layout, allocated once at load:
//   weights  one buffer; per layer the Q, K and V projection rows stacked into
//            one [n_embd + 2 kv] x n_embd Q8_0 matrix (and their biases into
//            one vector), gate and up rows interleaved into one 2 n_ff x n_embd
//            matrix (row 2i gate_i, row 2i + 1 up_i), so a layer is 4 matrix
//            launches; rows keep the GGUF block bytes (34-byte Q8_0 blocks),
//            every matrix 256-byte aligned;
//   KV       mi_hip_kv (F32, [head_dim, n_head_kv, n_ctx] per layer);
//   acts     x [n_embd, T] (the residual stream), qkv [n_embd + 2 kv, T],
//            attention output [head_dim, n_head, T], gate/up pairs [2 n_ff, T],
//            Q8_0 activation blocks for the widest input, logits [n_vocab, T].
// Per layer: RMSNorm*w -> Q8_0 blocks (one kernel), QKV + bias (matrix
// epilogue), RoPE + K/V append (one kernel), attention (decode or prefill
// kernel), Q8_0 blocks of its output, O projection + residual (epilogue, in
// place), RMSNorm*w -> blocks, gate/up with SiLU(gate)*up -> blocks (the
// matrix kernel's epilogue for one column, a kernel of its own for several),
// down projection + residual. Then the final norm of the returned columns,
// the lm_head and an argmax on the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "attn_common.h"
#include "gguf.h"
#include "kernels.h"
#include "mi_hip_attn.h"
#include "mi_hip_qwen2.h"

#define MI_LIBM_HD __host__ __device__
#include "libm_ref.h"

namespace mi {
namespace {

__constant__ uint64_t kExpfTab[32] = MI_EXPF_TABLE;

constexpr int kNormThreads = 256;
constexpr int kNormMaxE = 8192;  // widest normalised row (LDS copy of one column)

// GET_ROWS of token_embd (src/ops_cpu.cpp:102-132): x[:, j] = row ids[j],
// dequantised as (float)q * fp16 scale for Q8_0.
__global__ void embed_kernel(const char* w, int64_t row_bytes, int type, const int32_t* ids,
                             float* x, int E) {
  const int j = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= E) return;
  const char* row = w + (int64_t)gload<int>(ids + j) * row_bytes;
  float v;
  if (type == kGgufTQ8_0) {
    const char* blk = row + 34 * (i / 32);
    const float d = (float)__builtin_bit_cast(_Float16, gload<unsigned short>(blk));
    v = (float)gload<signed char>(blk + 2 + i % 32) * d;
  } else if (type == kGgufTF16) {
    v = (float)__builtin_bit_cast(_Float16, gload<unsigned short>(row + 2 * i));
  } else {
    v = gload<float>(row + 4 * i);
  }
  gstore<float>(x + (int64_t)j * E + i, v);
}

// RMS_NORM then MUL by the weight (src/ops_cpu.cpp:143-170), quantised to
// Q8_0_ACT blocks. One workgroup per column: squares in parallel, their sum in
// the reference's order by one lane (so the scale is the reference's to the
// bit), then one thread per element, 32 lanes to a block.
__global__ __launch_bounds__(kNormThreads) void norm_q8_kernel(const float* x, int64_t x_ld,
                                                               const float* w, float eps, char* aq,
                                                               int64_t aq_ld, int E) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float sq[kNormMaxE];
  __shared__ float s_scale;
  const float* xr = x + (int64_t)blockIdx.x * x_ld;
  for (int i = threadIdx.x; i < E; i += kNormThreads) {
    const float v = gload<float>(xr + i);
    sq[i] = v * v;
  }
  __syncthreads();
  if (threadIdx.x == 0) s_scale = rms_scale(ordered_sum(sq, E), E, eps);
  __syncthreads();
  const float scale = s_scale;
  char* dst = aq + (int64_t)blockIdx.x * aq_ld;
  for (int i = threadIdx.x; i < E; i += kNormThreads) {  // E % 32 == 0: whole 32-lane groups
    float d;
    const int q = q8_lane_quant((gload<float>(xr + i) * scale) * gload<float>(w + i), d);
    if ((i & 31) == 0) gstore<float>(dst + 36 * (i / 32), d);
    gstore<signed char>(dst + 36 * (i / 32) + 4 + (i & 31), (signed char)q);
  }
}

// SILU(gate) * up (src/ops_cpu.cpp:134-141, 167-170), quantised to Q8_0_ACT
// blocks from the interleaved gate/up pairs; one thread per element, 32 lanes
// to a block. silu(x) = x / (1 +
// expf(-x)) with the host C library's expf (libm_ref.h), so every value is the
// engine's.
__global__ void silu_mul_q8_kernel(const float* gu, int64_t gu_ld, int F, char* aq, int64_t aq_ld,
                                   int T) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)T * F) return;  // T * F % 32 == 0: whole 32-lane groups leave together
  const int64_t col = idx / F;
  const int e = (int)(idx - col * F);
  const float g = gload<float>(gu + col * gu_ld + 2 * e);
  const float y = (g / (1.0f + expf_ref(-g, kExpfTab))) * gload<float>(gu + col * gu_ld + 2 * e + 1);
  float d;
  const int q = q8_lane_quant(y, d);
  char* blk = aq + col * aq_ld + 36 * (e / 32);
  if ((e & 31) == 0) gstore<float>(blk, d);
  gstore<signed char>(blk + 4 + (e & 31), (signed char)q);
}

// mi_qwen2_sample_greedy (src/model_qwen2.cpp:690-700): starting from index 0,
// an index replaces the best only if its value is strictly greater. So the
// result is the first index of the largest non-NaN value when v[0] is not NaN,
// and 0 when it is (nothing compares greater than NaN). Two launches: each of
// kArgmaxParts workgroups scans one contiguous chunk (float4 loads, several in
// flight per lane) for its first largest non-NaN value; one wave merges the
// chunk results in chunk order (larger value, then smaller index).
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kArgmaxParts = 128;
constexpr int kArgmaxThreads = 256;
struct ArgBest {
  float v;
  int i;  // -1: no candidate yet
};
__device__ inline ArgBest arg_better(ArgBest a, ArgBest b) {
  if (b.i < 0) return a;
  if (a.i < 0 || b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}
__device__ inline ArgBest arg_wave(ArgBest b) {
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const ArgBest o{__shfl_xor(b.v, off), __shfl_xor(b.i, off)};
    b = arg_better(b, o);
  }
  return b;
}
__global__ __launch_bounds__(kArgmaxThreads) void argmax_part_kernel(const float* v, int n, int vec, float* pv,
                                                                     int* pi) {
  __shared__ ArgBest sb[kArgmaxThreads / kWave];
  const int chunk = ((n + kArgmaxParts - 1) / kArgmaxParts + 3) & ~3;  // a multiple of 4 elements
  const int b0 = min(n, (int)blockIdx.x * chunk), b1 = min(n, b0 + chunk);
  ArgBest best{0.f, -1};
  auto take = [&](float x, int i) {
    if (!(x != x) && (best.i < 0 || x > best.v)) best = ArgBest{x, i};
  };
  // float4 loads when v is 16-byte aligned (chunks start at multiples of 4)
  const int n4 = vec ? (b1 - b0) / 4 : 0;
  for (int j0 = threadIdx.x; j0 < n4; j0 += 4 * kArgmaxThreads) {
    f32x4 q[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u * kArgmaxThreads;
      q[u] = j < n4 ? gload<f32x4>(v + b0 + 4 * j) : f32x4{NAN, NAN, NAN, NAN};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) take(q[u][c], b0 + 4 * (j0 + u * kArgmaxThreads) + c);
  }
  for (int i = b0 + 4 * n4 + threadIdx.x; i < b1; i += kArgmaxThreads) take(gload<float>(v + i), i);
  best = arg_wave(best);
  if ((threadIdx.x & (kWave - 1)) == 0) sb[threadIdx.x / kWave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kArgmaxThreads / kWave; ++k) best = arg_better(best, sb[k]);
    gstore<float>(pv + blockIdx.x, best.v);
    gstore<int>(pi + blockIdx.x, best.i);
  }
}
__global__ __launch_bounds__(kWave) void argmax_final_kernel(const float* v, const float* pv, const int* pi,
                                                               int32_t* out) {
  ArgBest best{0.f, -1};
  for (int k = threadIdx.x; k < kArgmaxParts; k += kWave) best = arg_better(best, ArgBest{pv[k], pi[k]});
  best = arg_wave(best);
  if (threadIdx.x == 0) {
    const float v0 = gload<float>(v);
    gstore<int>(out, (v0 != v0 || best.i < 0) ? 0 : best.i);
  }
}

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace
}  // namespace mi

struct mi_hip_qwen2 {
  mi_hip_qwen2_hparams hp{};
  int n_ctx = 0, max_tokens = 0;
  int kvd = 0;  // n_head_kv * head_dim
  struct Layer {
    const float* attn_norm;
    const char* wqkv;
    const float* bqkv;
    const char* wo;
    const float* ffn_norm;
    const char* wgu;
    const char* wdown;
  };
  std::vector<Layer> layers;
  const char* tok_embd = nullptr;
  int tok_type = 0;
  int64_t tok_row_bytes = 0;
  const float* out_norm = nullptr;
  const char* lm_head = nullptr;
  int64_t row_e = 0, row_f = 0;  // Q8_0 bytes of an n_embd / n_ff wide row
  char* wbuf = nullptr;
  size_t wbytes = 0;
  mi_hip_kv* kv = nullptr;
  char* abuf = nullptr;
  size_t abytes = 0;
  float *x = nullptr, *qkv = nullptr, *ao = nullptr, *gu = nullptr, *logits = nullptr;
  char* aq = nullptr;
  int32_t *ids = nullptr, *next = nullptr;
  int32_t* gen = nullptr;      // greedy ids of a device-resident generation loop (n_ctx + 1)
  float* arg_v = nullptr;      // argmax: one (value, index) per chunk
  int32_t* arg_i = nullptr;
  int32_t *h_ids = nullptr, *h_next = nullptr, *h_gen = nullptr;  // pinned staging
  float* rope_cs = nullptr;  // (cos, sin) of every (position < n_ctx, pair), from the host's libm
  int attn_mode = MI_HIP_QWEN2_ATTN_REFERENCE_ORDER;  // FUSED when n_ctx > kExactMaxKeys
  hipStream_t stream = nullptr;
  bool timing = false;
  std::vector<hipEvent_t> ev;
  double attn_ms = 0, fwd_ms = 0;
  int64_t n_calls = 0;
};

namespace {

using mi::rt_fail;

int load_fail(mi_hip_qwen2* m, int rc);

#define Q2_TRY(expr, what)                                     \
  do {                                                         \
    hipError_t e_ = (expr);                                    \
    if (e_ != hipSuccess) return mi::rt_hip_fail(e_, what);    \
  } while (0)

int check_tensor(const mi::GgufFile& f, const std::string& name, uint32_t type, int64_t ne0,
                 int64_t ne1, const mi::GgufTensor** out) {
  const mi::GgufTensor* t = f.find_tensor(name.c_str());
  if (!t) return rt_fail(MI_HIP_E_INVALID, ("missing weight tensor: " + name).c_str());
  if (t->ne[0] != ne0 || t->ne[1] != ne1 || t->ne[2] != 1 || t->ne[3] != 1)
    return rt_fail(MI_HIP_E_INVALID, ("unexpected shape of " + name).c_str());
  if (type != UINT32_MAX && t->type != type)
    return rt_fail(MI_HIP_E_UNSUPPORTED,
                   ("tensor " + name + ": type " + std::to_string(t->type) +
                    (type == mi::kGgufTQ8_0 ? " (projections must be Q8_0)" : " (must be F32)"))
                       .c_str());
  *out = t;
  return MI_HIP_OK;
}

void destroy(mi_hip_qwen2* m) {
  if (!m) return;
  if (!m->wbuf && !m->kv && !m->abuf && !m->stream) {  // failed before touching the device
    delete m;
    return;
  }
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  for (hipEvent_t e : m->ev) (void)hipEventDestroy(e);
  if (m->kv) mi_hip_kv_destroy(m->kv);
  mi::rt_free(m->wbuf, m->wbytes);
  mi::rt_free(m->abuf, m->abytes);
  if (m->h_ids) (void)hipHostFree(m->h_ids);
  if (m->h_next) (void)hipHostFree(m->h_next);
  if (m->h_gen) (void)hipHostFree(m->h_gen);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

int load_fail(mi_hip_qwen2* m, int rc) {
  destroy(m);
  return rc;
}

int load_model(const char* path, int32_t n_ctx, int32_t max_tokens, mi_hip_qwen2* m) {
  mi::GgufFile f;
  std::string err;
  if (!f.open(path, &err)) return rt_fail(MI_HIP_E_INVALID, err.c_str());
  uint32_t E, L, H, Hkv, F, ctx_train;
  float base, eps;
  auto need_u32 = [&](const char* k, uint32_t* v) { return f.get_u32(k, v); };
  if (!need_u32("qwen2.embedding_length", &E) || !need_u32("qwen2.block_count", &L) ||
      !need_u32("qwen2.attention.head_count", &H) || !need_u32("qwen2.attention.head_count_kv", &Hkv) ||
      !need_u32("qwen2.feed_forward_length", &F) || !need_u32("qwen2.context_length", &ctx_train) ||
      !f.get_f32("qwen2.rope.freq_base", &base) ||
      !f.get_f32("qwen2.attention.layer_norm_rms_epsilon", &eps))
    return rt_fail(MI_HIP_E_INVALID, "qwen2 hparams: missing or wrong-typed key");
  if (H == 0 || E % H || Hkv == 0 || H % Hkv)
    return rt_fail(MI_HIP_E_INVALID, "qwen2 hparams: inconsistent head counts");
  const int hd = (int)(E / H);
  if (hd != 64 && hd != 128) return rt_fail(MI_HIP_E_UNSUPPORTED, "head_dim must be 64 or 128");
  if (E % 32 || F % 32 || E > (uint32_t)mi::kNormMaxE)
    return rt_fail(MI_HIP_E_UNSUPPORTED, "n_embd and n_ff must be multiples of 32 (n_embd <= 8192)");
  const mi::GgufTensor* te = f.find_tensor("token_embd.weight");
  if (!te || te->ne[0] != E || te->ne[2] != 1 || te->ne[3] != 1)
    return rt_fail(MI_HIP_E_INVALID, "missing or malformed token_embd.weight");
  if (te->ne[1] > INT32_MAX) return rt_fail(MI_HIP_E_UNSUPPORTED, "vocabulary too large");
  m->hp = {(int32_t)te->ne[1], (int32_t)E, (int32_t)L, (int32_t)H, (int32_t)Hkv, (int32_t)F,
           hd, (int32_t)ctx_train, base, eps};
  m->kvd = hd * (int)Hkv;
  if (n_ctx <= 0) return rt_fail(MI_HIP_E_INVALID, "n_ctx must be positive");
  m->n_ctx = n_ctx;
  if (n_ctx > mi::kExactMaxKeys) m->attn_mode = MI_HIP_QWEN2_ATTN_FUSED;
  m->max_tokens = max_tokens > 0 ? std::min(max_tokens, n_ctx) : n_ctx;
  const int64_t V = m->hp.n_vocab;
  m->row_e = E / 32 * 34;
  m->row_f = F / 32 * 34;

  // weights: collect (source, bytes) pieces in device order. The stacked Q
  // and K rows (and their biases) are permuted within each head so that a
  // RoPE pair, dims j and j + head_dim/2, are adjacent rows (2j, 2j + 1): the
  // matrix kernel's epilogue then rotates them in place; staged in host
  // memory, one copy per matrix.
  struct Piece { const uint8_t* src; size_t bytes; size_t off; };
  std::vector<Piece> pieces;
  std::vector<std::vector<uint8_t>> staged;
  size_t off = 0;
  auto place = [&](std::initializer_list<const mi::GgufTensor*> ts) {
    const size_t start = off;
    for (const mi::GgufTensor* t : ts) {
      pieces.push_back({t->data, t->nbytes, off});
      off += t->nbytes;
    }
    off = mi::align256(off);
    return start;
  };
  auto place_rope_rows = [&](std::initializer_list<const mi::GgufTensor*> ts, int64_t perm_rows, size_t rb) {
    size_t total = 0;
    for (const mi::GgufTensor* t : ts) total += t->nbytes;
    std::vector<uint8_t> buf(total);
    size_t o = 0;
    for (const mi::GgufTensor* t : ts) {
      std::memcpy(buf.data() + o, t->data, t->nbytes);
      o += t->nbytes;
    }
    std::vector<uint8_t> out(buf);  // rows of rb bytes (a weight row, or one bias element)
    for (int64_t r = 0; r < perm_rows; ++r)
      std::memcpy(out.data() + r * rb, buf.data() + mi::q8_unperm_row(r, hd, perm_rows) * rb, rb);
    staged.push_back(std::move(out));
    const size_t start = off;
    pieces.push_back({staged.back().data(), total, off});
    off = mi::align256(off + total);
    return start;
  };
  // two matrices of rb-byte rows interleaved row by row (the first's row i
  // at 2i, the second's at 2i + 1)
  auto place_pair_rows = [&](const mi::GgufTensor* a, const mi::GgufTensor* b, size_t rb) {
    const size_t rows = a->nbytes / rb;
    std::vector<uint8_t> out(a->nbytes + b->nbytes);
    for (size_t r = 0; r < rows; ++r) {
      std::memcpy(out.data() + 2 * r * rb, a->data + r * rb, rb);
      std::memcpy(out.data() + (2 * r + 1) * rb, b->data + r * rb, rb);
    }
    staged.push_back(std::move(out));
    const size_t start = off;
    pieces.push_back({staged.back().data(), staged.back().size(), off});
    off = mi::align256(off + staged.back().size());
    return start;
  };
  const mi::GgufTensor *on, *ow = nullptr;
  int rc;
  if ((rc = check_tensor(f, "output_norm.weight", mi::kGgufTF32, E, 1, &on))) return rc;
  if (f.find_tensor("output.weight")) {
    if ((rc = check_tensor(f, "output.weight", mi::kGgufTQ8_0, E, V, &ow))) return rc;
  } else if (te->type != mi::kGgufTQ8_0) {
    return rt_fail(MI_HIP_E_UNSUPPORTED, "a tied lm_head (token_embd.weight) must be Q8_0");
  }
  struct LayerOff { size_t an, qkv, bqkv, o, fn, gu, down; };
  std::vector<LayerOff> lo(L);
  const size_t tok_off = place({te});
  const size_t on_off = place({on});
  const size_t ow_off = ow ? place({ow}) : tok_off;
  for (uint32_t l = 0; l < L; ++l) {
    const std::string b = "blk." + std::to_string(l) + ".";
    const mi::GgufTensor *an, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *fn, *wg, *wu, *wd;
    if ((rc = check_tensor(f, b + "attn_norm.weight", mi::kGgufTF32, E, 1, &an)) ||
        (rc = check_tensor(f, b + "attn_q.weight", mi::kGgufTQ8_0, E, E, &wq)) ||
        (rc = check_tensor(f, b + "attn_q.bias", mi::kGgufTF32, E, 1, &bq)) ||
        (rc = check_tensor(f, b + "attn_k.weight", mi::kGgufTQ8_0, E, m->kvd, &wk)) ||
        (rc = check_tensor(f, b + "attn_k.bias", mi::kGgufTF32, m->kvd, 1, &bk)) ||
        (rc = check_tensor(f, b + "attn_v.weight", mi::kGgufTQ8_0, E, m->kvd, &wv)) ||
        (rc = check_tensor(f, b + "attn_v.bias", mi::kGgufTF32, m->kvd, 1, &bv)) ||
        (rc = check_tensor(f, b + "attn_output.weight", mi::kGgufTQ8_0, E, E, &wo)) ||
        (rc = check_tensor(f, b + "ffn_norm.weight", mi::kGgufTF32, E, 1, &fn)) ||
        (rc = check_tensor(f, b + "ffn_gate.weight", mi::kGgufTQ8_0, E, F, &wg)) ||
        (rc = check_tensor(f, b + "ffn_up.weight", mi::kGgufTQ8_0, E, F, &wu)) ||
        (rc = check_tensor(f, b + "ffn_down.weight", mi::kGgufTQ8_0, F, E, &wd)))
      return rc;
    lo[l] = {place({an}), place_rope_rows({wq, wk, wv}, E + m->kvd, (size_t)m->row_e),
             place_rope_rows({bq, bk, bv}, E + m->kvd, sizeof(float)),
             place({wo}), place({fn}), place_pair_rows(wg, wu, (size_t)m->row_e), place({wd})};
  }
  // everything above is host-side validation; the device is touched from here on
  if ((rc = mi::rt_bind())) return rc;
  void* p = nullptr;
  if ((rc = mi::rt_alloc(&p, off, "qwen2 weights"))) return rc;
  m->wbuf = static_cast<char*>(p);
  m->wbytes = off;
  for (const Piece& pc : pieces)
    Q2_TRY(hipMemcpy(m->wbuf + pc.off, pc.src, pc.bytes, hipMemcpyHostToDevice), "weight upload");
  m->tok_embd = m->wbuf + tok_off;
  m->tok_type = (int)te->type;
  m->tok_row_bytes = (int64_t)te->row_bytes;
  m->out_norm = reinterpret_cast<const float*>(m->wbuf + on_off);
  m->lm_head = m->wbuf + ow_off;
  m->layers.resize(L);
  for (uint32_t l = 0; l < L; ++l) {
    auto fp = [&](size_t o) { return reinterpret_cast<const float*>(m->wbuf + o); };
    m->layers[l] = {fp(lo[l].an), m->wbuf + lo[l].qkv, fp(lo[l].bqkv), m->wbuf + lo[l].o,
                    fp(lo[l].fn), m->wbuf + lo[l].gu, m->wbuf + lo[l].down};
  }

  // KV cache
  mi_hip_kv_desc kd{(int32_t)L, n_ctx, (int32_t)Hkv, hd, (int32_t)H, MI_TYPE_F32};
  if ((rc = mi_hip_kv_create(&kd, &m->kv))) return rc;

  // activations
  const int64_t T = m->max_tokens;
  const int64_t qkv_rows = E + 2 * m->kvd;
  const int64_t widest = std::max<int64_t>(E, F);
  size_t a = 0;
  const size_t ox = a; a = mi::align256(a + 4 * E * T);
  const size_t oqkv = a; a = mi::align256(a + 4 * qkv_rows * T);
  const size_t oao = a; a = mi::align256(a + 4 * E * T);
  const size_t ogu = a; a = mi::align256(a + 4 * 2 * (int64_t)F * T);
  const size_t oaq = a; a = mi::align256(a + (widest / 32) * 36 * T);
  const size_t olog = a; a = mi::align256(a + 4 * V * T);
  const size_t oids = a; a = mi::align256(a + 4 * T);
  const size_t onext = a; a = mi::align256(a + 4);
  const size_t ogen = a; a = mi::align256(a + 4 * ((size_t)n_ctx + 1));
  const size_t oarg = a; a = mi::align256(a + 8 * mi::kArgmaxParts);
  const size_t ocs = a; a = mi::align256(a + 4 * 2 * (size_t)n_ctx * (hd / 2));
  if ((rc = mi::rt_alloc(&p, a, "qwen2 activations"))) return rc;
  m->abuf = static_cast<char*>(p);
  m->abytes = a;
  m->x = reinterpret_cast<float*>(m->abuf + ox);
  m->qkv = reinterpret_cast<float*>(m->abuf + oqkv);
  m->ao = reinterpret_cast<float*>(m->abuf + oao);
  m->gu = reinterpret_cast<float*>(m->abuf + ogu);
  m->aq = m->abuf + oaq;
  m->logits = reinterpret_cast<float*>(m->abuf + olog);
  m->ids = reinterpret_cast<int32_t*>(m->abuf + oids);
  m->next = reinterpret_cast<int32_t*>(m->abuf + onext);
  m->gen = reinterpret_cast<int32_t*>(m->abuf + ogen);
  m->arg_v = reinterpret_cast<float*>(m->abuf + oarg);
  m->arg_i = reinterpret_cast<int32_t*>(m->abuf + oarg + 4 * mi::kArgmaxParts);
  m->rope_cs = reinterpret_cast<float*>(m->abuf + ocs);
  {
    // the engine's angles (src/ops_cpu.cpp:287-291): freq = powf(base, -(2p)/n_dims),
    // theta = (float)pos * freq, then the C library's cosf and sinf
    std::vector<float> cs(2 * (size_t)n_ctx * (hd / 2));
    for (int pos = 0; pos < n_ctx; ++pos)
      for (int pr = 0; pr < hd / 2; ++pr) {
        const float freq = std::pow(base, -(float)(2 * pr) / (float)hd);
        const float theta = (float)pos * freq;
        cs[2 * ((size_t)pos * (hd / 2) + pr)] = std::cos(theta);
        cs[2 * ((size_t)pos * (hd / 2) + pr) + 1] = std::sin(theta);
      }
    Q2_TRY(hipMemcpy(m->rope_cs, cs.data(), 4 * cs.size(), hipMemcpyHostToDevice), "rope table upload");
  }
  Q2_TRY(hipHostMalloc((void**)&m->h_ids, 4 * T, hipHostMallocDefault), "hipHostMalloc");
  Q2_TRY(hipHostMalloc((void**)&m->h_next, 4, hipHostMallocDefault), "hipHostMalloc");
  Q2_TRY(hipHostMalloc((void**)&m->h_gen, 4 * ((size_t)n_ctx + 1), hipHostMallocDefault), "hipHostMalloc");
  Q2_TRY(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "hipStreamCreate");
  m->ev.resize(2 * L);
  for (hipEvent_t& e : m->ev) Q2_TRY(hipEventCreate(&e), "hipEventCreate");
  return MI_HIP_OK;
}

// The activation of a projection: Q8_0_ACT blocks already in m->aq, or F32
// columns x (x_ld floats apart) to quantise, after RMS_NORM * norm_w if set.
struct Act {
  const float* x;
  const float* norm_w;
};

int quantize_cols(const mi_hip_qwen2* m, const float* src, int64_t ne0, int64_t cols, char* dst);

// dst[:, j] (+)= W . act[:, j] for j < m_cols. Decode-sized calls take the
// streaming matrix kernel with the norm / quantisation as its prologue (one
// launch); the others run the norm or quantize kernel into m->aq first.
// With swiglu_out (rows in gate/up pairs), one column is written as the
// Q8_0_ACT blocks of SiLU(gate) * up at swiglu_out when the matrix kernel's
// epilogue takes the shape (*swiglued says whether it did; otherwise dst holds
// the pairs).
int proj(const mi_hip_qwen2* m, const char* w, int64_t row_bytes, int64_t n, int64_t k, Act act,
         int64_t m_cols, float* dst, int64_t dst_ld, const float* add, int64_t add_ld,
         const mi::RopeEpi* rope = nullptr, bool* roped = nullptr, char* swiglu_out = nullptr,
         bool* swiglued = nullptr) {
  mi::Q8MulMat p{};
  p.w = w;
  p.a = m->aq;
  p.dst = reinterpret_cast<char*>(dst);
  p.w_nb1 = row_bytes;
  p.a_nb1 = k / 32 * 36;
  p.dst_nb0 = 4;
  p.dst_nb1 = 4 * dst_ld;
  p.k = k;
  p.n = n;
  p.m = m_cols;
  p.add = reinterpret_cast<const char*>(add);
  p.add_nb0 = add ? 4 : 0;
  p.add_nb1 = 4 * add_ld;
  if (act.x) {
    p.x = act.x;
    p.x_ld = k;
    p.norm_w = act.norm_w;
    p.eps = m->hp.rms_eps;
    if (!mi::q8_ring_form(p)) {
      p.x = nullptr;
      p.norm_w = nullptr;
      if (act.norm_w) {
        hipLaunchKernelGGL(mi::norm_q8_kernel, dim3((unsigned)m_cols), dim3(mi::kNormThreads), 0, m->stream,
                           act.x, k, act.norm_w, m->hp.rms_eps, m->aq, p.a_nb1, (int)k);
        Q2_TRY(hipGetLastError(), "norm launch");
      } else {
        int rc = quantize_cols(m, act.x, k, m_cols, m->aq);
        if (rc) return rc;
      }
    }
  }
  if (rope) {
    // the stacked Q/K rows are stored permuted: rotated in the epilogue when
    // the streaming form runs a single column, else put back in natural order
    if (p.x && m_cols == 1 && mi::q8_ring_form(p)) {
      p.rope_on = 1;
      p.rope = *rope;
    } else {
      p.perm_hd = rope->hd;
      p.perm_rows = (int64_t)rope->n_q + rope->n_kv;
    }
    if (roped) *roped = p.rope_on != 0;
  }
  if (swiglu_out && m_cols == 1) {
    p.swiglu_out = swiglu_out;
    if (!mi::q8_swiglu_out_ok(p, mi::rt_n_cu())) p.swiglu_out = nullptr;
  }
  if (swiglued) *swiglued = p.swiglu_out != nullptr;
  hipError_t e = mi::launch_mul_mat_q8_0(p, mi::rt_n_cu(), m->stream);
  return e == hipSuccess ? MI_HIP_OK : mi::rt_hip_fail(e, "qwen2 mul_mat launch");
}

int quantize_cols(const mi_hip_qwen2* m, const float* src, int64_t ne0, int64_t cols, char* dst) {
  mi::Q8Quantize p{};
  p.src = reinterpret_cast<const char*>(src);
  p.dst = dst;
  p.src_nb[0] = 4;
  p.src_nb[1] = 4 * ne0;
  p.src_nb[2] = p.src_nb[3] = 4 * ne0 * cols;
  p.dst_nb[0] = 1;
  p.dst_nb[1] = ne0 / 32 * 36;
  p.dst_nb[2] = p.dst_nb[3] = p.dst_nb[1] * cols;
  p.ne0 = ne0;
  p.ne1 = cols;
  p.ne2 = 1;
  p.rows = cols;
  hipError_t e = mi::launch_quantize_q8_0_act(p, m->stream);
  return e == hipSuccess ? MI_HIP_OK : mi::rt_hip_fail(e, "qwen2 quantize launch");
}

// Enqueues one forward pass on the model's stream, nothing waited for: the T
// token ids are read from device memory (ids_dev), the logits of the returned
// positions land in m->logits and the greedy id of the last one in next_dev.
// timed: bracket every layer's attention with the model's events.
int enqueue_forward(mi_hip_qwen2* m, const int32_t* ids_dev, int T, int n_past, bool last_only,
                    int32_t* next_dev, bool timed) {
  const mi_hip_qwen2_hparams& hp = m->hp;
  const int E = hp.n_embd, F = hp.n_ff, hd = hp.head_dim, H = hp.n_head;
  const int64_t qkv_rows = E + 2 * m->kvd;
  const int64_t ab_f = F / 32 * 36;
  hipStream_t st = m->stream;
  int rc;
  hipLaunchKernelGGL(mi::embed_kernel, dim3((E + 255) / 256, T), dim3(256), 0, st, m->tok_embd,
                     m->tok_row_bytes, m->tok_type, ids_dev, m->x, E);
  Q2_TRY(hipGetLastError(), "embed launch");
  const float scale = 1.0f / std::sqrt((float)hd);
  for (int l = 0; l < hp.n_layer; ++l) {
    const mi_hip_qwen2::Layer& w = m->layers[l];
    const size_t nb[3] = {4, 4 * (size_t)hd, 4 * (size_t)qkv_rows};
    void* kc = nullptr;
    void* vc = nullptr;
    int64_t cne[4];
    size_t cnb[4];
    if ((rc = mi_hip_kv_view(m->kv, l, 0, &kc, cne, cnb)) || (rc = mi_hip_kv_view(m->kv, l, 1, &vc, cne, cnb)))
      return rc;
    mi::RopeEpi re{};
    re.cs = m->rope_cs;
    re.q_out = m->qkv;
    re.k_row = static_cast<char*>(kc) + (int64_t)n_past * (int64_t)cnb[2];
    re.v_row = static_cast<char*>(vc) + (int64_t)n_past * (int64_t)cnb[2];
    re.c_s1 = (int64_t)cnb[1];
    re.pos = n_past;
    re.hd = hd;
    re.n_q = E;
    re.n_kv = m->kvd;
    bool roped = false;
    if ((rc = proj(m, w.wqkv, m->row_e, qkv_rows, E, {m->x, w.attn_norm}, T, m->qkv, qkv_rows, w.bqkv, 0, &re,
                   &roped)))
      return rc;
    if (!roped) {
      // RoPE on Q and K in place, K and V appended at positions n_past.. (one launch)
      mi::RopeAppend ra{};
      ra.q = reinterpret_cast<const char*>(m->qkv);
      ra.q_out = reinterpret_cast<char*>(m->qkv);
      ra.k = reinterpret_cast<const char*>(m->qkv + E);
      ra.v = reinterpret_cast<const char*>(m->qkv + E + m->kvd);
      void* kd = nullptr;
      int64_t ne[4];
      size_t cnb[4];
      if ((rc = mi_hip_kv_view(m->kv, l, 0, &kd, ne, cnb))) return rc;
      ra.k_cache = static_cast<char*>(kd);
      if ((rc = mi_hip_kv_view(m->kv, l, 1, &kd, ne, cnb))) return rc;
      ra.v_cache = static_cast<char*>(kd);
      for (int i = 0; i < 3; ++i) ra.q_nb[i] = ra.qo_nb[i] = ra.k_nb[i] = ra.v_nb[i] = (int64_t)nb[i];
      ra.c_s1 = (int64_t)cnb[1];
      ra.c_s2 = (int64_t)cnb[2];
      ra.n_tokens = T;
      ra.n_head = H;
      ra.n_head_kv = hp.n_head_kv;
      ra.head_dim = hd;
      ra.n_past = n_past;
      ra.n_dims = hd;
      ra.cs = m->rope_cs;
      Q2_TRY(mi::launch_rope_append(ra, false, st), "rope append launch");
    }
    mi_hip_attn_args aa{};
    aa.kv = m->kv;
    aa.layer = l;
    aa.q = m->qkv;
    for (int i = 0; i < 3; ++i) aa.q_nb[i] = nb[i];
    aa.out = m->ao;
    aa.out_nb[0] = 4;
    aa.out_nb[1] = 4 * (size_t)hd;
    aa.out_nb[2] = 4 * (size_t)E;
    aa.n_head = H;
    aa.n_rep = H / hp.n_head_kv;
    aa.n_past = n_past;
    aa.n_tokens = T;
    aa.scale = scale;
    aa.stream = st;
    if (timed) Q2_TRY(hipEventRecord(m->ev[2 * l], st), "hipEventRecord");
    if (m->attn_mode == MI_HIP_QWEN2_ATTN_REFERENCE_ORDER) {
      void* kd = nullptr;
      void* vd = nullptr;
      int64_t ne[4];
      size_t knb[4], vnb[4];
      if ((rc = mi_hip_kv_view(m->kv, l, 0, &kd, ne, knb)) || (rc = mi_hip_kv_view(m->kv, l, 1, &vd, ne, vnb)))
        return rc;
      mi::ExactAttn ea{};
      ea.q = reinterpret_cast<const char*>(m->qkv);
      ea.k = static_cast<const char*>(kd);
      ea.v = static_cast<const char*>(vd);
      ea.out = reinterpret_cast<char*>(m->ao);
      ea.q_s1 = (int64_t)nb[1];
      ea.q_s2 = (int64_t)nb[2];
      ea.k_s1 = (int64_t)knb[1];
      ea.k_s2 = (int64_t)knb[2];
      ea.v_s1 = (int64_t)vnb[1];
      ea.v_s2 = (int64_t)vnb[2];
      ea.o_s1 = 4 * (int64_t)hd;
      ea.o_s2 = 4 * (int64_t)E;
      ea.n_head = H;
      ea.n_rep = H / hp.n_head_kv;
      ea.n_past = n_past;
      ea.n_tokens = T;
      ea.head_dim = hd;
      ea.scale = scale;
      Q2_TRY(mi::launch_attn_exact(ea, st), "reference-order attention launch");
    } else if ((rc = mi_hip_attn_fwd(&aa))) {
      return rc;
    }
    if (timed) Q2_TRY(hipEventRecord(m->ev[2 * l + 1], st), "hipEventRecord");
    if ((rc = proj(m, w.wo, m->row_e, E, E, {m->ao, nullptr}, T, m->x, E, m->x, E))) return rc;
    bool swiglued = false;
    if ((rc = proj(m, w.wgu, m->row_e, 2 * (int64_t)F, E, {m->x, w.ffn_norm}, T, m->gu, 2 * (int64_t)F,
                   nullptr, 0, nullptr, nullptr, m->aq, &swiglued)))
      return rc;
    if (!swiglued) {
      const int64_t nel = (int64_t)T * F;
      hipLaunchKernelGGL(mi::silu_mul_q8_kernel, dim3((unsigned)((nel + 255) / 256)), dim3(256), 0, st,
                         m->gu, 2 * (int64_t)F, F, m->aq, ab_f, T);
      Q2_TRY(hipGetLastError(), "silu launch");
    }
    if ((rc = proj(m, w.wdown, m->row_f, E, F, {nullptr, nullptr}, T, m->x, E, m->x, E))) return rc;
  }
  const int first = last_only ? T - 1 : 0;
  const int n_out = T - first;
  if ((rc = proj(m, m->lm_head, m->row_e, hp.n_vocab, E, {m->x + (int64_t)first * E, m->out_norm}, n_out,
                 m->logits, hp.n_vocab, nullptr, 0)))
    return rc;
  const float* last_row = m->logits + (int64_t)(n_out - 1) * hp.n_vocab;
  hipLaunchKernelGGL(mi::argmax_part_kernel, dim3(mi::kArgmaxParts), dim3(mi::kArgmaxThreads), 0, st, last_row,
                     hp.n_vocab, (reinterpret_cast<uintptr_t>(last_row) & 15) == 0 ? 1 : 0, m->arg_v, m->arg_i);
  Q2_TRY(hipGetLastError(), "argmax launch");
  hipLaunchKernelGGL(mi::argmax_final_kernel, dim3(1), dim3(mi::kWave), 0, st, last_row, m->arg_v, m->arg_i, next_dev);
  Q2_TRY(hipGetLastError(), "argmax merge launch");
  return MI_HIP_OK;
}

int forward(mi_hip_qwen2* m, const int32_t* tokens, int T, int n_past, bool last_only,
            float* logits_out, int32_t* next_id) {
  const mi_hip_qwen2_hparams& hp = m->hp;
  hipStream_t st = m->stream;
  std::memcpy(m->h_ids, tokens, 4 * (size_t)T);
  Q2_TRY(hipMemcpyAsync(m->ids, m->h_ids, 4 * (size_t)T, hipMemcpyHostToDevice, st), "ids upload");
  int rc = enqueue_forward(m, m->ids, T, n_past, last_only, m->next, m->timing);
  if (rc) return rc;
  const int n_out = last_only ? 1 : T;
  Q2_TRY(hipMemcpyAsync(m->h_next, m->next, 4, hipMemcpyDeviceToHost, st), "next id copy");
  if (logits_out)
    Q2_TRY(hipMemcpyAsync(logits_out, m->logits, 4 * (size_t)hp.n_vocab * n_out, hipMemcpyDeviceToHost, st),
           "logits copy");
  Q2_TRY(hipStreamSynchronize(st), "hipStreamSynchronize");
  if (next_id) *next_id = *m->h_next;
  if (m->timing) {
    for (int l = 0; l < hp.n_layer; ++l) {
      float ms = 0;
      Q2_TRY(hipEventElapsedTime(&ms, m->ev[2 * l], m->ev[2 * l + 1]), "hipEventElapsedTime");
      m->attn_ms += ms;
    }
  }
  return MI_HIP_OK;
}

// The reference CLI's greedy loop (src/main.cpp:462-495) with every step on
// the device: the prompt's forward call, then one forward call per further
// id, each step's embedding reading the id the previous step's argmax wrote
// (m->gen[i - 1]), so steps follow one another on the stream without a host
// round trip; the ids come back in one copy at the end. Same ids as calling
// forward once per token.
int generate(mi_hip_qwen2* m, const int32_t* prompt, int n_prompt, int n_predict, int32_t* out_ids,
             int32_t* n_out) {
  hipStream_t st = m->stream;
  std::memcpy(m->h_ids, prompt, 4 * (size_t)n_prompt);
  Q2_TRY(hipMemcpyAsync(m->ids, m->h_ids, 4 * (size_t)n_prompt, hipMemcpyHostToDevice, st), "ids upload");
  int rc = enqueue_forward(m, m->ids, n_prompt, 0, true, m->gen, false);
  if (rc) return rc;
  int n = n_predict > 0 ? 1 : 0, n_past = n_prompt;
  for (; n < n_predict && n_past < m->n_ctx; ++n, ++n_past)
    if ((rc = enqueue_forward(m, m->gen + n - 1, 1, n_past, true, m->gen + n, false))) return rc;
  if (n > 0) Q2_TRY(hipMemcpyAsync(m->h_gen, m->gen, 4 * (size_t)n, hipMemcpyDeviceToHost, st), "ids copy");
  Q2_TRY(hipStreamSynchronize(st), "hipStreamSynchronize");
  std::memcpy(out_ids, m->h_gen, 4 * (size_t)n);
  *n_out = n;
  return MI_HIP_OK;
}

}  // namespace

extern "C" {

int mi_hip_qwen2_load(const char* gguf_path, int32_t n_ctx, int32_t max_tokens, mi_hip_qwen2** out) {
  if (!gguf_path || !out) return rt_fail(MI_HIP_E_INVALID, "gguf_path and out must be non-NULL");
  *out = nullptr;
  int rc;
  mi_hip_qwen2* m = new (std::nothrow) mi_hip_qwen2();
  if (!m) return rt_fail(MI_HIP_E_NOMEM, "host allocation failed");
  if ((rc = load_model(gguf_path, n_ctx, max_tokens, m))) return load_fail(m, rc);
  *out = m;
  return MI_HIP_OK;
}

int mi_hip_qwen2_free(mi_hip_qwen2* model) {
  if (!model) return MI_HIP_OK;
  int rc = mi::rt_bind();
  if (rc) return rc;
  destroy(model);
  return MI_HIP_OK;
}

int mi_hip_qwen2_get_hparams(const mi_hip_qwen2* model, mi_hip_qwen2_hparams* out) {
  if (!model || !out) return rt_fail(MI_HIP_E_INVALID, "model and out must be non-NULL");
  *out = model->hp;
  return MI_HIP_OK;
}

int mi_hip_qwen2_forward(mi_hip_qwen2* model, const int32_t* tokens, int32_t n_tokens,
                         int32_t n_past, int32_t last_logits_only, float* logits_out,
                         int32_t* next_id) {
  if (!model || !tokens) return rt_fail(MI_HIP_E_INVALID, "model and tokens must be non-NULL");
  if (n_tokens <= 0 || n_tokens > model->max_tokens)
    return rt_fail(MI_HIP_E_INVALID, ("n_tokens must be in [1, " + std::to_string(model->max_tokens) + "]").c_str());
  if (n_past < 0 || (int64_t)n_past + n_tokens > model->n_ctx)
    return rt_fail(MI_HIP_E_INVALID, ("positions exceed n_ctx = " + std::to_string(model->n_ctx)).c_str());
  for (int i = 0; i < n_tokens; ++i)
    if (tokens[i] < 0 || tokens[i] >= model->hp.n_vocab)
      return rt_fail(MI_HIP_E_INVALID, ("token id " + std::to_string(tokens[i]) + " outside the vocabulary").c_str());
  int rc = mi::rt_bind();
  if (rc) return rc;
  const auto t0 = std::chrono::steady_clock::now();
  rc = forward(model, tokens, n_tokens, n_past, last_logits_only != 0, logits_out, next_id);
  if (rc) return rc;
  model->fwd_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  model->n_calls++;
  return MI_HIP_OK;
}

int mi_hip_qwen2_generate(mi_hip_qwen2* model, const int32_t* prompt, int32_t n_prompt, int32_t n_predict,
                          int32_t* out_ids, int32_t* n_out) {
  if (!model || !prompt || !n_out || (n_predict > 0 && !out_ids))
    return rt_fail(MI_HIP_E_INVALID, "model, prompt, n_out (and out_ids when n_predict > 0) must be non-NULL");
  *n_out = 0;
  if (n_prompt <= 0 || n_prompt > model->max_tokens)
    return rt_fail(MI_HIP_E_INVALID, ("n_prompt must be in [1, " + std::to_string(model->max_tokens) + "]").c_str());
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] < 0 || prompt[i] >= model->hp.n_vocab)
      return rt_fail(MI_HIP_E_INVALID, ("token id " + std::to_string(prompt[i]) + " outside the vocabulary").c_str());
  int rc = mi::rt_bind();
  if (rc) return rc;
  return generate(model, prompt, n_prompt, n_predict, out_ids, n_out);
}

int mi_hip_qwen2_set_attention(mi_hip_qwen2* model, int32_t mode) {
  if (!model) return rt_fail(MI_HIP_E_INVALID, "model is NULL");
  if (mode != MI_HIP_QWEN2_ATTN_FUSED && mode != MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
    return rt_fail(MI_HIP_E_INVALID, "unknown attention mode");
  if (mode == MI_HIP_QWEN2_ATTN_REFERENCE_ORDER && model->n_ctx > mi::kExactMaxKeys)
    return rt_fail(MI_HIP_E_UNSUPPORTED, "reference-order attention covers n_ctx <= 32768");
  model->attn_mode = mode;
  return MI_HIP_OK;
}

int mi_hip_qwen2_set_timing(mi_hip_qwen2* model, int32_t enable) {
  if (!model) return rt_fail(MI_HIP_E_INVALID, "model is NULL");
  model->timing = enable != 0;
  model->attn_ms = model->fwd_ms = 0;
  model->n_calls = 0;
  return MI_HIP_OK;
}

int mi_hip_qwen2_get_timing(mi_hip_qwen2* model, double* attn_ms, double* forward_ms, int64_t* n_calls) {
  if (!model) return rt_fail(MI_HIP_E_INVALID, "model is NULL");
  if (attn_ms) *attn_ms = model->attn_ms;
  if (forward_ms) *forward_ms = model->fwd_ms;
  if (n_calls) *n_calls = model->n_calls;
  return MI_HIP_OK;
}

}  // extern "C"
