/*
 * mi_hip_qwen2.h -- C ABI of a Qwen2 decoder resident on one MI355X (gfx950):
 * the engine around the attention path, so that a whole generation step runs
 * on the device with the attention nodes on the fused HIP kernels.
 *
 * What it replaces (the reference engine's model API, src/model_qwen2.h):
 *   mi_qwen2_model_load     src/model_qwen2.cpp:466-537  (GGUF -> weights)
 *   mi_kv_cache_init        src/model_qwen2.cpp:548-590  (KV cache + arenas)
 *   mi_qwen2_forward        src/model_qwen2.cpp:609-688  (one forward call)
 *   mi_qwen2_sample_greedy  src/model_qwen2.cpp:690-700  (argmax, first index)
 *   mi_qwen2_model_free / mi_kv_cache_free
 * The graph of one forward call is the reference's (src/model_qwen2.cpp:
 * 133-191 per layer, 213-234 around them): embedding lookup, per layer
 * RMSNorm * weight, Q/K/V projections + bias, RoPE, K/V append, fused
 * attention, output projection + residual, RMSNorm * weight, SiLU(gate) * up,
 * down projection + residual; final RMSNorm * weight and the (tied) lm_head.
 *
 * Numerics: Q8_0 products, activation quantisation, RMSNorm (summed in the
 * reference's order), the embedding dequantisation, the additions, RoPE (its
 * cosines and sines tabulated at load by the host's own cosf/sinf) and SiLU
 * (the host's expf, restated bit for bit) are bit-exact with the reference;
 * the attention is bit-exact in MI_HIP_QWEN2_ATTN_REFERENCE_ORDER mode and
 * within 1e-4 in the default fused mode.
 *
 * Conventions as in mi_hip_attn.h: int status (MI_HIP_OK == 0), message in
 * mi_hip_last_error(); mi_hip_init must have been called. Host pointers are
 * ordinary host memory. Calls are synchronous (they return once the step's
 * results are in host memory).
 */
#ifndef MI_HIP_QWEN2_H
#define MI_HIP_QWEN2_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mi_hip_qwen2 mi_hip_qwen2;

/* src/model_qwen2.h's mi_qwen2_hparams, read from the GGUF keys
 * qwen2.* (src/model_qwen2.cpp:426-463). */
typedef struct mi_hip_qwen2_hparams {
  int32_t n_vocab;
  int32_t n_embd;
  int32_t n_layer;
  int32_t n_head;
  int32_t n_head_kv;
  int32_t n_ff;
  int32_t head_dim;
  int32_t n_ctx_train;
  float rope_freq_base;
  float rms_eps;
} mi_hip_qwen2_hparams;

/* Loads a Qwen2 GGUF v3 file (Q8_0 projection weights; F32 norms and
 * biases; token_embd F32, F16 or Q8_0, and Q8_0 when it doubles as the
 * lm_head), copies the weights to the device and allocates, once, the F32 KV
 * cache for n_ctx positions and the activations for forward calls of up to
 * max_tokens tokens (0: n_ctx). Nothing is allocated by later calls.
 * Replaces mi_qwen2_model_load + mi_kv_cache_init. */
int mi_hip_qwen2_load(const char* gguf_path, int32_t n_ctx, int32_t max_tokens,
                      mi_hip_qwen2** out);
int mi_hip_qwen2_free(mi_hip_qwen2* model);

int mi_hip_qwen2_get_hparams(const mi_hip_qwen2* model, mi_hip_qwen2_hparams* out);

/* One forward call over tokens[0..n_tokens) at positions n_past.. (the KV
 * cache must hold positions [0, n_past) from earlier calls), as
 * mi_qwen2_forward with params.last_logits_only = last_logits_only:
 *   logits_out (host, may be NULL): n_vocab floats per returned position
 *     (the last one only, or all n_tokens);
 *   next_id (host, may be NULL): the greedy token of the last position
 *     (mi_qwen2_sample_greedy: the first index of the maximum).
 * Token ids are checked against [0, n_vocab). */
int mi_hip_qwen2_forward(mi_hip_qwen2* model, const int32_t* tokens, int32_t n_tokens,
                         int32_t n_past, int32_t last_logits_only, float* logits_out,
                         int32_t* next_id);

/* Greedy generation as the reference CLI runs it (src/main.cpp:462-495): one
 * forward call over prompt[0..n_prompt) at position 0, then one call per
 * further id, each on the id before it, until n_predict ids (the first from
 * the prompt call) or until the cache's n_ctx positions are used. The ids
 * (n_predict at most, count in *n_out) are the same as those of calling
 * mi_hip_qwen2_forward once per token; here each step's embedding reads the
 * previous step's greedy id from device memory, so the steps run back to back
 * on the device without a host round trip between them, and the ids come
 * back in one copy. Every call starts from position 0. Per-layer attention
 * timing does not apply to it. No counterpart in the reference (its loop
 * samples on the host between calls). */
int mi_hip_qwen2_generate(mi_hip_qwen2* model, const int32_t* prompt, int32_t n_prompt,
                          int32_t n_predict, int32_t* out_ids, int32_t* n_out);

/* Attention kernels of the forward calls.
 *   MI_HIP_QWEN2_ATTN_FUSED: the throughput kernels of mi_hip_attn.h
 *     (split-KV decode, MFMA prefill; within 1e-4 of the reference ops, so
 *     greedy ids follow the reference engine's until a near-tie argmax).
 *     The default when n_ctx > 32768.
 *   MI_HIP_QWEN2_ATTN_REFERENCE_ORDER (the default for n_ctx <= 32768): one
 *     wave per (token, head) running the
 *     reference's own operation order (src/ops_cpu.cpp:304-410: ordered dot
 *     products and sums, the C library's expf), bit-identical to the engine;
 *     cost linear in the context per row. With it every step of a forward call
 *     is bit-identical to the reference engine's, so greedy token ids match
 *     exactly (the Q8_0 activation rounding turns any ulp of difference into
 *     a visibly different trajectory after tens of steps). n_ctx <= 32768.
 * No counterpart in the reference. */
#define MI_HIP_QWEN2_ATTN_FUSED 0
#define MI_HIP_QWEN2_ATTN_REFERENCE_ORDER 1
int mi_hip_qwen2_set_attention(mi_hip_qwen2* model, int32_t mode);

/* Per-call timing (off by default): when enabled, each forward call brackets
 * every layer's attention launch with HIP events. Totals since the last reset:
 * attention kernel milliseconds, wall milliseconds of the forward calls, and
 * the number of calls. No counterpart in the reference (its --bench times
 * whole calls, src/main.cpp:392-419). */
int mi_hip_qwen2_set_timing(mi_hip_qwen2* model, int32_t enable);
int mi_hip_qwen2_get_timing(mi_hip_qwen2* model, double* attn_ms, double* forward_ms,
                            int64_t* n_calls);

#ifdef __cplusplus
}
#endif

#endif /* MI_HIP_QWEN2_H */
