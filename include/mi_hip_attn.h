/*
 * mi_hip_attn.h -- C ABI of the MI355X (gfx950) batched GQA attention
 * backend for the mini-infer engine.
 *
 * What it replaces: the three CPU graph ops
 *   MI_OP_ATTN_QK   src/ops_cpu.cpp:356-380  (scores  S[i,j,h] = K[:,h/n_rep,i].Q[:,h,j])
 *   MI_OP_SOFTMAX   src/ops_cpu.cpp:304-346  (causal, scaled, per (j,h) row)
 *   MI_OP_ATTN_KQV  src/ops_cpu.cpp:386-410  (O[o,h,j] = sum_t V[o,h/n_rep,t].P[t,j,h])
 * plus the KV cache that feeds them (src/model_qwen2.cpp:557-596, the K/V
 * append CPY nodes of src/model_qwen2.cpp:156-159) and the per-node dispatch
 * point of the executor (src/ops_cpu.cpp:481-530, src/threadpool.cpp:171-180).
 *
 * Conventions
 *   - Every function returns an int status (MI_HIP_OK == 0). It never throws
 *     and never aborts on bad arguments; the message of the last failure on
 *     the calling thread is returned by mi_hip_last_error().
 *   - Layouts are the engine's: Q and O are [head_dim, n_head, n_tokens], the
 *     K and V caches are [head_dim, n_head_kv, n_ctx] per layer, ne[0]
 *     innermost, strides in bytes. Q head h reads KV head h / n_rep: GQA is an
 *     index mapping, no K/V row is ever copied per head.
 *   - Pointers named "device" must be device (HBM) addresses; "host" pointers
 *     are ordinary host memory.
 *   - `stream` is a hipStream_t passed as void*; NULL means the null stream.
 *     Calls enqueue work and return; the caller synchronises the stream.
 */
#ifndef MI_HIP_ATTN_H
#define MI_HIP_ATTN_H

#include <stddef.h>
#include <stdint.h>

#include "mi_tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define MI_HIP_OK 0
#define MI_HIP_E_INVALID 1     /* an argument is out of range or inconsistent */
#define MI_HIP_E_NODEVICE 2    /* no usable gfx950 device */
#define MI_HIP_E_RUNTIME 3     /* a HIP runtime call failed */
#define MI_HIP_E_NOMEM 4       /* device allocation refused (or over the limit) */
#define MI_HIP_E_UNSUPPORTED 5 /* valid request outside what the kernels cover */
#define MI_HIP_E_STATE 6       /* called before mi_hip_init / on a dead object */
#define MI_HIP_E_LOST 7        /* a decode launch lost a record (its group's output is NaN) */

/* ---- library lifetime -------------------------------------------------- */

/* Selects `device` for this library and checks it is gfx950.
 * Counterpart of the engine's one-time setup in mi_kv_cache_init
 * (src/model_qwen2.cpp:557-596); idempotent for the same device. */
int mi_hip_init(int device);

/* Releases library-owned device memory (the default workspace). KV caches
 * and workspaces must have been destroyed by the caller first. */
int mi_hip_shutdown(void);

/* Thread-local text of the last failure ("" if none). */
const char* mi_hip_last_error(void);

/* Writes sizeof(mi_tensor), offsetof(type, ne, nb, op, op_params, src, data,
 * view_src, view_offs, n_children, flags, name, extra) and sizeof(mi_cgraph)
 * into out[0..14] (n >= 15) so a caller can verify it shares the layout of
 * src/tensor.h:122-160 and src/graph.h:19-47. */
int mi_hip_abi_layout(size_t* out, int n);

/* ---- device allocation accounting -------------------------------------- */

/* The engine forbids steady-state allocation (tests/test_zero_alloc.cpp).
 * Every device allocation this library makes goes through one counter. */
typedef struct mi_hip_alloc_stats {
  uint64_t n_malloc;
  uint64_t n_free;
  uint64_t bytes_live;
  uint64_t bytes_peak;
} mi_hip_alloc_stats;

int mi_hip_get_alloc_stats(mi_hip_alloc_stats* out);

/* Caps the library's live device bytes (0 = no cap). An allocation that
 * would exceed the cap fails with MI_HIP_E_NOMEM before calling HIP. */
int mi_hip_set_alloc_limit(uint64_t bytes);

/* ---- decode workspace ---------------------------------------------------- */

/* The split-KV decode kernel's scratch: one partial-result record per
 * workgroup, per-group counters (dynamic sub-tile claims, merge election,
 * arrivals) and status words. Launches that share a workspace must be
 * ordered (one stream, or synchronised); launches on different workspaces may
 * run concurrently. Every KV cache owns one (mi_hip_kv_workspace); callers
 * that attend over explicit tensors create their own, or fall back to the
 * library's default workspace (created by mi_hip_init, shared by every call
 * that names none). No counterpart in the reference: its CPU kernels need no
 * scratch beyond the graph allocator's arena (src/gallocr.cpp). */
typedef struct mi_hip_workspace mi_hip_workspace;

typedef struct mi_hip_workspace_desc {
  int32_t n_head_kv;  /* KV heads of the problems it serves */
  int32_t n_head;     /* Q heads (multiple of n_head_kv) */
  int32_t head_dim;   /* 64 or 128 */
} mi_hip_workspace_desc;

/* One device allocation covering any decode launch of up to 32 items of this
 * head shape (mi_hip_attn_decode_batch's limit per launch). */
int mi_hip_workspace_create(const mi_hip_workspace_desc* desc, mi_hip_workspace** out);
int mi_hip_workspace_destroy(mi_hip_workspace* ws);

typedef struct mi_hip_workspace_status {
  uint32_t early_fallbacks; /* early merges whose bounded wait ran out (results still exact) */
  uint32_t lost_groups;     /* groups whose output was set to NaN (never expected) */
} mi_hip_workspace_status;

/* Synchronises `stream`, reports the status words accumulated since the last
 * call and clears them. Returns MI_HIP_E_LOST if any group was lost (its
 * counters are then reset too), MI_HIP_OK otherwise. */
int mi_hip_workspace_check(mi_hip_workspace* ws, void* stream, mi_hip_workspace_status* out);

/* Rounds of polls an early merger makes before it falls back to the
 * last-arriver merge (default 4096). Tuning and tests; 0 makes every early
 * merge fall back. */
int mi_hip_workspace_set_poll_limit(mi_hip_workspace* ws, int32_t rounds);

/* Decode planner knobs (initialised from MI_HIP_DECODE_KPG, _EARLY, _SOLO and
 * _CLAIM at mi_hip_init): kpg > 0 forces that many workgroups per group (0:
 * planned); early = 0 disables the early merge, 1 uses it when every
 * workgroup of a launch fits on the device at once, 2 always; solo: groups
 * that one workgroup's ring covers in at most `solo` rounds get one
 * workgroup; claim: split groups whose waves each stream at least `claim`
 * ring rounds take sub-tiles from device counters (0: never). A negative
 * value keeps the current setting. Tuning and tests; no counterpart in the
 * reference. */
int mi_hip_decode_tuning(int32_t kpg, int32_t early, int32_t solo, int32_t claim);

/* Deterministic fused attention (on = 1, the default): every wave of the
 * decode and prefill kernels takes a fixed share of its workgroup's work, so
 * each output is the same bits on every run with the same inputs and launch
 * shape (the merges across waves and workgroups run in a fixed order). Off
 * (0): each wave takes the next piece of work from a counter, so a wave that
 * memory serves sooner takes more -- about 1% faster on the 24-layer
 * n_kv 4096 decode, with results that differ from run to run in the last
 * bits. Process-wide; takes effect for launches issued afterwards. No
 * counterpart in the reference (its CPU kernels are deterministic by
 * construction: src/ops_cpu.cpp:38-53). */
int mi_hip_set_deterministic(int32_t on);

/* Matrix cores of the prefill kernel's QK and PV products.
 *   MI_HIP_PREFILL_AUTO (the default): MI_HIP_PREFILL_F32 with an F32 cache,
 *     the split form below with an F16 cache (whose f16 products are exact
 *     in the cache operand); within the 1e-4 bar at any score magnitude
 *     either way.
 *   MI_HIP_PREFILL_F32: v_mfma_f32_32x32x2f32 (float products, as the
 *     reference's ops; an F16 cache widened to float), within the 1e-4 bar
 *     at any score magnitude.
 *   MI_HIP_PREFILL_SPLIT_BF16: with an F32 cache every float operand is split
 *     into a pair of bf16 (hi = round(x), lo = round(x - hi),
 *     |x - hi - lo| <= 2^-17 |x|) and each product is lo.hi + hi.lo + hi.hi
 *     on v_mfma_f32_32x32x16_bf16 with float accumulation: ~2^-16 relative
 *     error per product, three bf16 products at 16x the FP32 matrix rate,
 *     within the 1e-4 bar only while scale * |q| * |k| stays small (N(0,1)
 *     inputs with q and k scaled by up to 2). With an F16 cache the cache
 *     operand is used as it is and Q and the probabilities are split into
 *     f16 pairs (~2^-22 relative; a wave whose |q| exceeds 2^14 scales its
 *     queries by a power of two first): two v_mfma_f32_32x32x16_f16 per
 *     product step, within the bar at any score magnitude.
 * Process-wide. No counterpart in the reference. */
#define MI_HIP_PREFILL_F32 0
#define MI_HIP_PREFILL_SPLIT_BF16 1
#define MI_HIP_PREFILL_AUTO 2
int mi_hip_set_prefill_mode(int32_t mode);

/* Products of the decode kernel (one query row per head).
 *   MI_HIP_DECODE_MATRIX: QK and PV on the matrix cores (16x16 MFMAs; head
 *     columns padded to 16). F32 cache operands are split into bf16 pairs as
 *     in MI_HIP_PREFILL_SPLIT_BF16 (lo.hi + hi.lo + hi.hi); an F16 cache is
 *     used as it is, with Q and the probabilities split into f16 pairs (a
 *     head whose |q| exceeds 2^14 is scaled by a power of two first). ~1e-5
 *     relative per product.
 *   MI_HIP_DECODE_VALU: float multiply-adds on the vector units (exact
 *     float products).
 *   MI_HIP_DECODE_STREAM: float multiply-adds on the vector units in the
 *     streaming kernel (K/V straight into registers, each group's parts
 *     merged by the last to arrive), for head_dim 64 or 128 and groups that
 *     span several workgroups; other launches take MI_HIP_DECODE_VALU.
 *   MI_HIP_DECODE_AUTO (the default): the vector units (MI_HIP_DECODE_VALU)
 *     for an F32 cache; for an F16 cache the matrix cores, except for short
 *     launches whose heads can be split between workgroups so that each
 *     wave streams fewer than 4 sub-tiles of 16 positions (the split is a
 *     vector-unit form, faster there).
 * The split bf16 pairs of the matrix form carry ~2^-16 relative error per
 * product into the scores, so with an F32 cache it stays within the 1e-4 bar
 * only while scale * |q| * |k| stays small (N(0,1) inputs with q and k
 * scaled by up to 2); the other forms are within it at any magnitude.
 * Process-wide. No counterpart in the reference. */
#define MI_HIP_DECODE_VALU 0
#define MI_HIP_DECODE_MATRIX 1
#define MI_HIP_DECODE_AUTO 2
#define MI_HIP_DECODE_STREAM 3
int mi_hip_set_decode_mode(int32_t mode);

/* ---- device-resident KV cache ------------------------------------------ */

typedef struct mi_hip_kv mi_hip_kv;

typedef struct mi_hip_kv_desc {
  int32_t n_layer;
  int32_t n_ctx;
  int32_t n_head_kv;
  int32_t head_dim;  /* 64 or 128 */
  int32_t n_head;    /* Q heads (multiple of n_head_kv); sizes staging */
  int32_t type;      /* MI_TYPE_F32 or MI_TYPE_F16 cache elements */
} mi_hip_kv_desc;

/* One device allocation holding every layer's K and V as
 * [head_dim, n_head_kv, n_ctx] (position-major, the layout of
 * src/model_qwen2.cpp:564-577), plus the host-node staging buffer (sized for
 * n_ctx) and the cache's own decode workspace (covering a decode launch of up
 * to 32 items of this head shape). Nothing is allocated afterwards.
 * Replaces mi_kv_cache_init's host KV context (src/model_qwen2.cpp:564-577). */
int mi_hip_kv_create(const mi_hip_kv_desc* desc, mi_hip_kv** out);
int mi_hip_kv_destroy(mi_hip_kv* kv);

/* The cache's own decode workspace (owned by the cache; do not destroy). */
int mi_hip_kv_workspace(mi_hip_kv* kv, mi_hip_workspace** out);

/* Device view of one layer's cache: which = 0 for K, 1 for V. Fills the
 * device address and the engine-style ne[4]/nb[4]. */
int mi_hip_kv_view(mi_hip_kv* kv, int layer, int which, void** data, int64_t ne[4],
                   size_t nb[4]);

/* Writes n_tokens F32 rows src[head_dim, n_head_kv, n_tokens] (byte strides
 * src_nb[0..2]) into positions [pos0, pos0 + n_tokens) of layer `layer`'s
 * K (which = 0) or V (which = 1); F16 caches round to nearest even.
 * src_on_device = 0 for a host source, 1 for a device source.
 * This is the CPY-into-kv_write_view node (src/model_qwen2.cpp:99-103,
 * 156-159; src/ops_cpu.cpp:446-460). Host sources are synchronous. */
int mi_hip_kv_write(mi_hip_kv* kv, int layer, int which, int pos0, int n_tokens,
                    const float* src, const size_t src_nb[3], int src_on_device,
                    void* stream);

/* Associates the engine's host KV tensor (the persistent leaf whose
 * view_src-flattened views the CPY nodes write through, and which the
 * ATTN_QK/ATTN_KQV nodes read as src[1]) with a layer of `kv`, for
 * mi_hip_compute_forward. Keyed by the tensor's address, never by its
 * `extra` field (the engine's allocator rewrites `extra` every step,
 * src/gallocr.cpp:120-121). */
int mi_hip_kv_bind(mi_hip_kv* kv, int layer, int which, const mi_tensor* host_kv);

/* ---- fused attention ---------------------------------------------------- */

typedef struct mi_hip_attn_args {
  /* K/V source: either a cache + layer (kv != NULL) ... */
  mi_hip_kv* kv;
  int32_t layer;
  /* ... or explicit device tensors [head_dim, n_head_kv, >= n_past+n_tokens]. */
  const void* k;
  const void* v;
  size_t k_nb[3];
  size_t v_nb[3];
  int32_t kv_type;   /* MI_TYPE_F32 / MI_TYPE_F16 (explicit tensors only) */
  int32_t head_dim;  /* explicit tensors only */
  int32_t n_head_kv; /* explicit tensors only */
  /* Queries: device [head_dim, n_head, n_tokens], byte strides q_nb. */
  const float* q;
  size_t q_nb[3];
  /* Output: device [head_dim, n_head, n_tokens], byte strides out_nb. */
  float* out;
  size_t out_nb[3];
  int32_t n_head;
  int32_t n_rep;    /* n_head / n_head_kv (op_params[1] of ATTN_QK) */
  int32_t n_past;   /* keys [0, n_past + j] visible to query j */
  int32_t n_tokens; /* 1 = decode kernel, > 1 = prefill kernel */
  float scale;      /* op_params[1] of SOFTMAX, 1/sqrt(head_dim) in the engine */
  void* stream;
  /* Decode scratch: this workspace if non-NULL, else kv's own, else the
   * library default (read from the first item of a batch). */
  mi_hip_workspace* ws;
} mi_hip_attn_args;

/* The whole ATTN_QK -> causal SOFTMAX -> ATTN_KQV triple in one pass that
 * never materialises scores or probabilities: the split-KV decode kernel when
 * n_tokens == 1, the MFMA prefill kernel otherwise. Equivalent to running
 * mi_compute_attn_qk, mi_compute_softmax and mi_compute_attn_kqv
 * (src/ops_cpu.cpp:304-410) on the nodes built by src/model_qwen2.cpp:169-172,
 * within floating-point tolerance. */
int mi_hip_attn_fwd(const mi_hip_attn_args* args);

/* The same triple in the reference's own operation order, so that the output
 * equals mi_compute_attn_qk -> mi_compute_softmax -> mi_compute_attn_kqv
 * (src/ops_cpu.cpp:304-410) on the nodes of src/model_qwen2.cpp:169-172 BIT
 * FOR BIT, not within tolerance: each score's dot product d ascending with
 * every product and sum rounded, the maximum, the host C library's expf, the
 * sum of the exponentials key by key, the correctly rounded 1 / sum, and each
 * output element's sum over the keys in order. The device engine's
 * MI_HIP_QWEN2_ATTN_REFERENCE_ORDER mode runs it. F32 cache only, head_dim 64
 * or 128, n_past + n_tokens <= 32768 (MI_HIP_E_UNSUPPORTED otherwise). The
 * ordered sums make a row's cost linear in its key count on one lane: a
 * parity path, slower than mi_hip_attn_fwd. */
int mi_hip_attn_fwd_reference_order(const mi_hip_attn_args* args);

/* n_items independent single-token decode problems of one shape (same
 * head_dim, n_head, n_rep, K/V element type; n_past may differ) in ONE
 * launch, e.g. many sequences' caches, or a stack of layers in a benchmark.
 * No counterpart in the reference (it runs one node per layer).
 * Decode launches take a fresh stamp on their workspace from the host at
 * every call, so a call on a stream under graph capture is refused with
 * MI_HIP_E_UNSUPPORTED (a replayed launch would reuse its stamp); the same
 * holds for every decode entry point. */
int mi_hip_attn_decode_batch(const mi_hip_attn_args* items, int n_items, void* stream);

/* mi_hip_attn_decode_batch for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc). No counterpart in
 * the reference. Like every decode entry point it is refused on a stream
 * under graph capture. It ignores the items' ws and
 * their caches' workspaces and uses a fixed 4 MB scratch array that each GPU
 * holds from library load until the process ends (at most 128 groups, i.e.
 * items x n_head_kv x head chunks, and records for ~460-900 workgroups); a
 * larger launch fails with MI_HIP_E_UNSUPPORTED. It calls no hipMalloc or
 * hipFree. Every call on one GPU shares that GPU's scratch: calls that
 * overlap on the device (different streams, unsynchronised) race and must
 * not be issued; calls ordered on one stream are safe. */
int mi_hip_attn_decode_batch_noalloc(const mi_hip_attn_args* items, int n_items, void* stream);

/* ---- node-level operators on device tensors ----------------------------- */
/*
 * Same signature idea as the engine's kernels (src/ops_cpu.h:3-12): the node
 * `dst` carries op, op_params and src[], and every tensor's `data` is a DEVICE
 * address. Strides are honoured as in mi_f32_ptr (src/ops_cpu.cpp:38-41).
 */

/* MI_OP_ATTN_QK (src/ops_cpu.cpp:356-380; builder src/graph.cpp:241-253). */
int mi_hip_op_attn_qk(mi_tensor* dst, void* stream);
/* MI_OP_SOFTMAX (src/ops_cpu.cpp:304-346; builder src/graph.cpp:156-163). */
int mi_hip_op_softmax(mi_tensor* dst, void* stream);
/* MI_OP_ATTN_KQV (src/ops_cpu.cpp:386-410; builder src/graph.cpp:263-273). */
int mi_hip_op_attn_kqv(mi_tensor* dst, void* stream);
/* The fused triple given its last node: dst is the ATTN_KQV node,
 * dst->src[0] the SOFTMAX node, dst->src[0]->src[0] the ATTN_QK node. */
int mi_hip_op_attn_fused(mi_tensor* dst, void* stream);

/* MI_OP_ROPE (src/ops_cpu.cpp:270-302; builder src/graph.cpp:146-154,
 * op_params n_past, n_dims, freq_base): rotary embedding of dst->src[0]
 * [head_dim, n_heads, n_tokens] into dst (may be the same memory), NEOX
 * halves (element p pairs with p + n_dims/2), token i at position n_past + i.
 * The frequencies base^(-2p/n_dims) are the host's powf values, as in the
 * engine; the angle's cosine and sine are computed on the device. n_dims must
 * be even, at most head_dim and at most 256. */
int mi_hip_op_rope(mi_tensor* dst, void* stream);

/* ---- the step after attention: Q8_0 matrix-vector products -------------- */

/* MI_OP_QUANTIZE_Q8_0 (src/ops_cpu.cpp:462-479, row quantizer
 * src/quant.cpp:188-210; builder src/graph.cpp:117-128): dst (type
 * MI_TYPE_Q8_0_ACT, blocks of a float scale and 32 int8) from an F32 src of
 * the same ne[], each row contiguous (nb[0] = 4), ne[0] a multiple of 32.
 * Bit-exact: amax/127 scale, round half to even, clamp to [-127, 127]. */
int mi_hip_op_quantize_q8_0(mi_tensor* dst, void* stream);

/* MI_OP_MUL_MAT with Q8_0 weights (src/ops_cpu.cpp:226-236; builder
 * src/graph.cpp:130-144): dst [n, m] F32 = src[0] (MI_TYPE_Q8_0 [k, n], GGUF
 * blocks, row i at nb[1] * i) times src[1] (MI_TYPE_Q8_0_ACT [k, m], column j
 * at nb[1] * j), e.g. the attention output projection. Bit-exact with the
 * reference's default dot product (src/quant_avx2.cpp:174-185). F32 and F16
 * weights are not handled here (MI_HIP_E_UNSUPPORTED). */
int mi_hip_op_mul_mat(mi_tensor* dst, void* stream);

/* ---- the step before attention: RoPE and the KV append, fused ---------- */

/* One layer's qh_rot = rope(qh); kh_rot = rope(kh); cpy(kh_rot -> cache K
 * rows [n_past, n_past + n_tokens)); cpy(vh -> cache V rows) of
 * src/model_qwen2.cpp:153-159, in one launch on device tensors, so Q, K and
 * V never pass through host memory. Shapes [head_dim, heads, n_tokens] with
 * byte strides nb[0..2] (q/q_out: n_head heads, k/v: the cache's n_head_kv).
 * q may be NULL (no Q); q_out may equal q. F16 caches round K and V to
 * nearest even, like mi_hip_kv_write. */
typedef struct mi_hip_rope_args {
  mi_hip_kv* kv;
  int32_t layer;
  int32_t n_past;
  int32_t n_tokens;
  int32_t n_dims;   /* rotated dims (even, <= head_dim), op_params[1] of ROPE */
  float freq_base;  /* op_params[2] of ROPE */
  int32_t n_head;   /* Q heads */
  const float* q;
  size_t q_nb[3];
  float* q_out;
  size_t q_out_nb[3];
  const float* k;
  size_t k_nb[3];
  const float* v;
  size_t v_nb[3];
  void* stream;
} mi_hip_rope_args;

int mi_hip_rope_append(const mi_hip_rope_args* args);

/* ---- executor hook for host-resident graphs ------------------------------ */

/* Plans one step's graph (call after the allocator assigned data, before
 * execution): marks every ATTN_QK -> SOFTMAX -> ATTN_KQV chain whose scores
 * and probabilities have no other reader as fused. Allocation-free. */
int mi_hip_graph_prepare(const mi_cgraph* graph);

/* Drop-in for the dispatch in mi_compute_forward (src/ops_cpu.cpp:481-530),
 * same (dst, ith, nth) contract as every engine kernel (src/ops_cpu.h:3-12)
 * and the executor's per-node barrier (src/threadpool.cpp:171-180).
 * Returns 1 if the node belongs to this backend (the caller then skips its CPU
 * kernel), 0 if it does not, -1 on error (see mi_hip_last_error). Only ith == 0
 * does work: it enqueues the node on the KV cache's stream and waits for it,
 * so the node's host output is complete before the caller's barrier. Nodes
 * handled: CPY into a bound KV tensor; ATTN_QK and SOFTMAX of a planned fused
 * chain (no-ops); ATTN_KQV of a planned fused chain (the fused launch). */
int mi_hip_compute_forward(mi_tensor* dst, int ith, int nth);

/* Host-resident attention nodes (opt-in, default off): with on = 1,
 * mi_hip_compute_forward also takes ATTN_QK, SOFTMAX and ATTN_KQV nodes that
 * are not part of a fused chain on a bound KV cache -- e.g. a model whose
 * head_dim the fused kernels do not cover (they take 64 and 128), so its
 * cache stays on the host -- and runs each on the node kernels (bit-exact
 * with src/ops_cpu.cpp:304-410): its sources are copied to a staging buffer
 * (grown, and therefore allocated, to the largest node seen), the node runs,
 * its output is copied back before the call returns. A correctness path for
 * such models, not a throughput one. Process-wide. No counterpart in the
 * reference. */
int mi_hip_set_host_nodes(int32_t on);

/* ---- read-bandwidth ceiling ---------------------------------------------- */

/* The device counterpart of tools/bench_memread.cpp (the engine's read-only
 * bandwidth ceiling: a load-and-accumulate pass, one reduced sum per worker,
 * no writes to the source): n_sums workgroups each sum one contiguous slice
 * of src[0, bytes) (float data) and write sums[w]; sum(sums) is the sum of
 * the buffer up to float rounding. src is device memory, 16-byte aligned,
 * bytes a multiple of 16; sums is device memory of n_sums floats, 1 <= n_sums
 * <= 65536. Timed by the caller on `stream`: bytes / kernel time is the
 * measured ceiling that the decode kernels are compared with. */
int mi_hip_memread(const void* src, size_t bytes, float* sums, int32_t n_sums, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_HIP_ATTN_H */
