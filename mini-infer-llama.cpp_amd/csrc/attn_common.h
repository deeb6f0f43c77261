// attn_common.h -- launch parameters and device helpers shared by the HIP
// attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Decode (one query token against n_kv cached positions).
// ---------------------------------------------------------------------------
constexpr int kDecodeMaxItems = 32;  // items per launch (they ride in kernarg)
constexpr int kDecodeTile = 64;      // positions per wave iteration (lane = position)
constexpr int kDecodeKStride = 68;   // LDS floats per staged K row (64 + 4 pad)
constexpr int kDecodeWaves = 4;      // waves per workgroup

// One independent decode problem. Byte strides; the head_dim axis of K, V, Q
// and O is contiguous.
struct DecodeItem {
  const char* k;
  const char* v;
  const float* q;
  float* out;
  int64_t k_s1, k_s2;  // K: bytes between heads, between positions
  int64_t v_s1, v_s2;
  int64_t q_s1;        // Q: bytes between heads
  int64_t o_s1;        // O: bytes between heads
  int32_t n_kv;        // keys [0, n_kv) are visible
  int32_t pad_;
};

struct DecodeParams {
  DecodeItem item[kDecodeMaxItems];
  int32_t n_items;
  int32_t n_rep;        // Q heads per KV head
  int32_t n_head_kv;
  int32_t n_chunks;     // head chunks per KV head (n_rep / G)
  int32_t splits;       // position splits per (item, head chunk)
  float scale_log2e;    // softmax scale * log2(e)
  float* part;          // split partials (splits > 1)
  unsigned* counter;    // arrival counters, one per (item, head chunk); self-resetting
};

// ---------------------------------------------------------------------------
// Prefill (n_tokens queries, causal).
// ---------------------------------------------------------------------------
constexpr int kPrefillRows = 32;   // queries per wave unit (MFMA N)
constexpr int kPrefillKeys = 32;   // keys per tile (MFMA M)
constexpr int kPrefillWaves = 4;

struct PrefillParams {
  const char* k;
  const char* v;
  const float* q;
  float* out;
  int64_t k_s1, k_s2, v_s1, v_s2;  // bytes
  int64_t q_s1, q_s2;              // bytes between heads, between tokens
  int64_t o_s1, o_s2;
  int32_t n_head, n_rep, n_past, n_tokens;
  int32_t chunk_tiles;   // key tiles per unit (C)
  int32_t n_qblocks;     // ceil(n_tokens / 32)
  int32_t units_per_head;
  int32_t n_units;       // n_head * units_per_head
  float scale_log2e;
  float* part;           // per-unit partials
  unsigned* counter;     // per (head, q-block); self-resetting
};

// Prefix sum sum_{t=1..x} ceil(t / c) in closed form.
__host__ __device__ inline int64_t ceil_prefix(int64_t x, int64_t c) {
  const int64_t a = x / c, b = x % c;
  return c * a * (a + 1) / 2 + b * (a + 1);
}

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
__device__ inline float wave_max(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
  return x;
}

__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Orders this wave's LDS accesses (the wave executes LDS operations in issue
// order; this stops the compiler from moving them across the point).
__device__ inline void wave_lds_fence() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

// Four consecutive cache elements as float4 (F32: one 16-byte load; F16: one
// 8-byte load widened exactly).
template <typename KT>
__device__ inline float4 load4(const char* p);

template <>
__device__ inline float4 load4<float>(const char* p) {
  return *reinterpret_cast<const float4*>(p);
}

template <>
__device__ inline float4 load4<_Float16>(const char* p) {
  const half4_t h = *reinterpret_cast<const half4_t*>(p);
  return make_float4((float)h.x, (float)h.y, (float)h.z, (float)h.w);
}

// Uniform (scalar-cache) view of a global buffer: loads through it with a
// wave-uniform address are issued as scalar loads into SGPRs.
typedef const __attribute__((address_space(4))) float* const_f32_ptr;

__device__ inline const_f32_ptr as_const(const float* p) {
  return (const_f32_ptr)(p);
}

}  // namespace mi
