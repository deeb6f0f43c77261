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
constexpr int kDecodeEarlyMax = 8;   // largest group merged by its first finisher
constexpr int kDecodeSub = 16;       // positions per sub-tile (one wave's unit of work)
constexpr int kDecodeWaves = 4;      // waves per workgroup (one per SIMD)

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
  int32_t spg;         // sub-tiles per group, ceil(n_kv / kDecodeSub) (host planning)
  int32_t wg0;         // first workgroup of this item
  int32_t kpg;         // workgroups per group
};

// Per-group counter block of the decode workspace (kCtrInts words, 256 bytes,
// so groups never share a cache line): the dynamic sub-tile claims, the early
// protocol's merger election, start count (plus the merger's give-up mark),
// late-part count and give-up point, and the team arrivals.
constexpr int kCtrInts = 64;
constexpr int kCtrClaim = 0;
constexpr int kCtrElect = 16;
constexpr int kCtrStarted = 17;
constexpr int kCtrLate = 18;
constexpr int kCtrGaveUpAt = 19;
constexpr int kCtrTeams = 32;  // team t arrives at word kCtrTeams + t (t < 32)
// Status words of a workspace: [0] early merges whose bounded wait ran out and
// that fell back to the last-arriver merge; [1] records never seen (the output
// of that group is NaN). Cleared by the host.
constexpr int kStatusWords = 4;

// Work decomposition. A group is (item, KV head g, head chunk hc): the G Q
// heads g*n_rep + hc*G .. + G - 1 that read KV head g. Each group is served by
// kpg workgroups of its item (workgroups wg0 + gl*kpg + part, part < kpg),
// which take the group's 16-position sub-tiles dynamically and leave one
// record each when kpg > 1.
struct DecodeParams {
  // Scalars first: the kernel reads them in one round of scalar loads.
  int32_t n_rep;        // Q heads per KV head
  int32_t n_head_kv;
  int32_t n_chunks;     // head chunks per KV head; chunk hc holds heads
                        // [hc n_rep / n_chunks, (hc + 1) n_rep / n_chunks)
  int32_t gpi;          // groups per item, n_head_kv * n_chunks
  int32_t n_wg;         // workgroups with work (records)
  int32_t early;        // groups of 2..kDecodeEarlyMax workgroups merged by their first finisher
  int32_t det;          // 1: each wave takes fixed sub-tiles (the same bits on every run)
  int32_t max_polls;    // the early merger's bounded wait (rounds of polls) before it falls back
  int32_t ctr_groups;   // groups one counter set covers
  int32_t clear_groups; // groups [0, clear_groups) of the other counter set to clear
  uint32_t epoch;       // launch stamp (nonzero, new for every launch on this workspace)
  int32_t rec_words;    // 64-bit words per record slot (the streaming kernel)
  float scale_log2e;    // softmax scale * log2(e)
  float* rec;           // one record per workgroup
  unsigned* cnt;        // two counter sets of ctr_groups * kCtrInts words: launch e uses set
                        // e & 1 (zero on entry) and clears set (e + 1) & 1 for the next launch
  unsigned* status;     // kStatusWords status words
  DecodeItem item[kDecodeMaxItems];  // grid row y serves item y
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
  int32_t n_qblocks;     // ceil(n_tokens / 32)
  int32_t lone;          // 1: the last query block has a workgroup of its own
  int32_t det;           // 1: each wave takes fixed units (the same bits on every run)
  float scale_log2e;
};

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) char lds_t;

// Raw (unswizzled, stride 0) buffer descriptor word 3 of the gfx9 family.
constexpr int kRawBufferWord3 = 0x00020000;

// Descriptor over [p, p + bytes): accesses whose per-lane offset (plus the
// instruction's constant offset) reaches bytes read zero and make no memory
// request. The scalar offset operand is not part of that range check.
__device__ inline rsrc_t make_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           kRawBufferWord3);
}

// Waits until at most N vector memory operations of this wave are in flight
// (they complete in issue order). Needed after buffer_load ... lds, which the
// compiler does not track.
template <int N>
__device__ inline void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier that waits only for this wave's LDS operations: unlike
// __syncthreads() it never makes the compiler drain vector-memory loads that
// are still in flight (a ring's LDS-direct requests keep streaming across it).
__device__ inline void wg_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Loads and stores through the global address space. Pointers that reach a
// kernel through LDS (a staged argument table) are otherwise generic, and a
// generic (flat) access counts against both the vector-memory and the LDS
// counters, so every later LDS wait would also wait for it.
template <typename T>
__device__ __forceinline__ T gload(const void* p) {
  typedef const __attribute__((address_space(1))) T gT;
  return *(gT*)p;
}
template <typename T>
__device__ __forceinline__ void gstore(void* p, T v) {
  typedef __attribute__((address_space(1))) T gT;
  *(gT*)p = v;
}

// Typed LDS accesses through the LDS address space (32-bit addresses).
template <typename T>
__device__ __forceinline__ T lds_load(const lds_t* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(p);
}
template <typename T>
__device__ __forceinline__ void lds_store(lds_t* p, T v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>(p) = v;
}
// 16 bytes per lane from r + voff into LDS at lds + 16 * lane (buffer_load ...
// lds). Kept out of templates: the host pass drops a kernel template whose
// body names the builtin directly.
__device__ inline void dma16(rsrc_t r, lds_t* lds, unsigned voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, 0, 0, 0);
}
// Cache-policy bit of a buffer access (gfx950 cpol): nontemporal, for data
// read once per launch (a KV cache stream), so that it does not displace what
// the caches hold for longer.
constexpr int kNt = 2;
__device__ inline void dma16_nt(rsrc_t r, lds_t* lds, unsigned voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, 0, 0, kNt);
}

// LDS rows of NSLOT 16-byte slots: logical slot j of row r is stored at
// physical slot j ^ swz(r), so 16 lanes reading one slot of 16 consecutive
// rows hit distinct banks.
template <int NSLOT>
__host__ __device__ constexpr int swz(int r) {
  return NSLOT >= 16 ? (r & 15) : ((r >> 1) & (NSLOT - 1));
}

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

// DPP lane moves (VALU, no LDS). Within each row of 16 lanes:
//   xor1 / xor2: quad_perm [1,0,3,2] / [2,3,0,1] (0xB1 / 0x4E); half_mirror:
//   i <-> 7-i; mirror: i <-> 15-i; row_ror:N (0x120 + N): lane i takes lane
//   (i + N) % 16; bcast<J>: lane J of the row to the whole row.
template <int CTRL>
__device__ inline float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
template <int J>
__device__ inline float row_bcast(float x) { return dpp_mov<0x150 + J>(x); }

// acc + bcast_J(q) * k in ONE instruction: v_fmac_f32 with a DPP row_newbcast
// source operand (lane J of each row of 16 supplies q to the whole row). The
// compiler does not form this itself (the accumulator is tied), hence asm.
// Callers never write q with a VALU instruction right before (q comes from a
// load), so the DPP source-read wait states are met.
template <int J>
__device__ inline float fmac_bcast(float acc, float q, float k) {
  asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
      : "+v"(acc)
      : "v"(q), "v"(k), "i"(J));
  return acc;
}

// Max over the 16 lanes of each row, left in every lane of the row.
__device__ inline float row_max16(float x) {
  x = fmaxf(x, dpp_mov<0xB1>(x));   // quad_perm [1,0,3,2]
  x = fmaxf(x, dpp_mov<0x4E>(x));   // quad_perm [2,3,0,1]
  x = fmaxf(x, dpp_mov<0x141>(x));  // row_half_mirror
  x = fmaxf(x, dpp_mov<0x140>(x));  // row_mirror
  return x;
}

// Max over the wave, wave-uniform result: rows by DPP, then the four row
// maxima through readlane (no LDS traffic).
__device__ inline float wave_max_dpp(float x) {
  x = row_max16(x);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

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

// ---------------------------------------------------------------------------
// Q8_0 activation blocks and the RMS norm scale, shared by the matrix kernels
// and the engine (the engine's arithmetic: src/quant.cpp:188-210 and
// src/ops_cpu.cpp:143-165).

// The RMS norm scale from the ordered sum of squares: mean = sum / E,
// 1 / sqrt(mean + eps), each a correctly rounded float operation (computed in
// double, whose single rounding to float is the float operation's).
__device__ inline float rms_scale(float sumsq, int E, float eps) {
  const float mean = (float)((double)sumsq / (double)E);
  const float root = (float)__builtin_sqrt((double)(mean + eps));
  return (float)(1.0 / (double)root);
}

// The ordered sum of n squares sq[0..n) (n % 4 == 0, 16-byte aligned), by one lane.
__device__ inline float ordered_sum(const float* sq, int n) {
#pragma clang fp contract(off)
  float s = 0.0f;
  const float4* q4 = reinterpret_cast<const float4*>(sq);
#pragma unroll 8
  for (int i = 0; i < n / 4; ++i) {
    const float4 v = q4[i];
    s = s + v.x;
    s = s + v.y;
    s = s + v.z;
    s = s + v.w;
  }
  return s;
}

// The same sum over the N floats at LDS byte address sq (N a multiple of
// 16; callers pad with +0.0, which leaves a sum of squares unchanged), for
// one lane. The reads are issued as asm two chunks of 16 values ahead of the
// additions, each chunk's wait tied to its registers: the chain of additions
// does not wait for LDS, and the compiler neither reorders the reads nor
// waits for LDS-direct requests elsewhere in LDS (it does not see the reads).
namespace sum_lds {
typedef float f32x4_t __attribute__((ext_vector_type(4)));
template <int C>
__device__ __forceinline__ void load(unsigned sq, f32x4_t (&d)[4]) {
  asm volatile(
      "ds_read_b128 %0, %4 offset:%5\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b128 %2, %4 offset:%7\n\t"
      "ds_read_b128 %3, %4 offset:%8"
      : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3])
      : "v"(sq), "n"(64 * C), "n"(64 * C + 16), "n"(64 * C + 32), "n"(64 * C + 48));
}
template <int K>
__device__ __forceinline__ void wait(f32x4_t (&d)[4]) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]) : "n"(K));
}
template <int C, int KC>
__device__ __forceinline__ void chunks(unsigned sq, f32x4_t (&b)[3][4], float& s) {
#pragma clang fp contract(off)
  if constexpr (C < KC) {
    if constexpr (C + 2 < KC) load<C + 2>(sq, b[(C + 2) % 3]);
    constexpr int later = KC - 1 - C < 2 ? KC - 1 - C : 2;  // chunks requested after this one
    wait<4 * later>(b[C % 3]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      s = s + b[C % 3][u].x;
      s = s + b[C % 3][u].y;
      s = s + b[C % 3][u].z;
      s = s + b[C % 3][u].w;
    }
    chunks<C + 1, KC>(sq, b, s);
  }
}
// s plus the N floats at LDS byte address sq, one rounded addition each, in order
template <int N>
__device__ __forceinline__ float run(unsigned sq, float s) {
  static_assert(N % 16 == 0 && 4 * N <= 65536, "whole chunks of 16, offsets in range");
  f32x4_t b[3][4];
  load<0>(sq, b[0]);
  if constexpr (N / 16 > 1) load<1>(sq, b[1]);
  chunks<0, N / 16>(sq, b, s);
  return s;
}
}  // namespace sum_lds

template <int N>
__device__ __forceinline__ float ordered_sum_lds(const lds_t* sq) {
  return sum_lds::run<N>((unsigned)(uintptr_t)sq, 0.0f);
}

// The same ordered sum of 8 * L non-negative floats at sq (LDS; callers pad
// with +0.0), formed by 8 waves together, every wave returning it. Segment j
// (floats jL .. jL + L - 1) belongs to wave j, which runs the segment's chain
// of additions from 64 start values at once, one per lane: the consecutive
// floats from 32 below g_j, the float nearest to the exact sum of the floats
// before the segment (a sum in double: it only places the candidates). The
// true start of segment j is the end of segment j - 1's chain from its own
// true start, so each wave then walks the segments in order, taking for each
// the lane whose start equals the running sum (non-negative floats are
// ordered like their bit patterns, so that lane is the bit difference), or,
// if the running sum is not among the 64 (a rounding drift of more than 32
// ulps from the exact prefix), continuing the chain itself. The result is
// the one-lane sum's to the bit, in about a quarter of its time. work: 8 * 8
// + 8 * 64 * 4 bytes of LDS, 16-byte aligned. Every wave of the workgroup
// calls it (two barriers).
// A wave's sum of one double per lane, on every lane, without the LDS pipe:
// quad and row rotations by DPP moves, then the four row sums by readlane
// (a fixed order, so every lane and every call gets the same bits).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double x) {
  const uint64_t b = __builtin_bit_cast(uint64_t, x);
  const unsigned lo = __builtin_bit_cast(unsigned, dpp_mov<CTRL>(__builtin_bit_cast(float, (unsigned)b)));
  const unsigned hi = __builtin_bit_cast(unsigned, dpp_mov<CTRL>(__builtin_bit_cast(float, (unsigned)(b >> 32))));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum_f64(double x) {
  x += dpp_f64<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_f64<0x4E>(x);   // quad_perm [2,3,0,1]: every lane holds its quad's sum
  x += dpp_f64<0x124>(x);  // row_ror:4
  x += dpp_f64<0x128>(x);  // row_ror:8: every lane holds its row's sum
  auto lane_val = [&](int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
  };
  return ((lane_val(0) + lane_val(16)) + lane_val(32)) + lane_val(48);
}

// The walk's way out when a running sum is not among a segment's candidates
// (kept out of line: it is rare).
template <int L>
__device__ __noinline__ float ordered_sum_continue(unsigned sq, float s) {
  return sum_lds::run<L>(sq, s);
}

template <int L>
__device__ float ordered_sum_lds_8waves(const lds_t* sq, lds_t* work, int wv, int lane) {
#pragma clang fp contract(off)
  static_assert(L % 16 == 0 && L <= 2 * kWave, "whole chunks of 16, at most two floats per lane");
  typedef double f64x2_t __attribute__((ext_vector_type(2)));
  const unsigned a_sq = (unsigned)(uintptr_t)sq;
  const unsigned a_q = (unsigned)(uintptr_t)work;  // 8 segment sums (double)
  const unsigned a_r = a_q + 64;                   // 8 x 64 chain ends
  const unsigned seg = a_sq + 4 * L * wv;
  // (LDS reads as asm: the compiler cannot tell these runtime addresses from
  // LDS-direct requests in flight elsewhere, and would wait for those)
  float v0 = 0.0f, v1 = 0.0f;
  asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %2 offset:256\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(v0), "=&v"(v1) : "v"(seg + 4 * lane));
  const double q = wave_sum_f64((lane < L ? (double)v0 : 0.0) + (lane + kWave < L ? (double)v1 : 0.0));
  if (lane == 0) lds_store<double>(work + 8 * wv, q);
  wg_barrier();
  f64x2_t q01, q23, q45, q67;  // work is 16-byte aligned
  asm volatile(
      "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:16\n\t"
      "ds_read_b128 %2, %4 offset:32\n\tds_read_b128 %3, %4 offset:48\n\ts_waitcnt lgkmcnt(0)"
      : "=&v"(q01), "=&v"(q23), "=&v"(q45), "=&v"(q67)
      : "v"(a_q));
  const double qs[8] = {q01.x, q01.y, q23.x, q23.y, q45.x, q45.y, q67.x, q67.y};
  // every segment's lowest candidate (the same on every wave)
  int base[8];
  double pre = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int gb = __builtin_bit_cast(int, (float)pre);
    base[j] = gb > 32 ? gb - 32 : 0;
    pre += qs[j];
  }
  int my_base = base[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) my_base = wv == j ? base[j] : my_base;
  const float end = sum_lds::run<L>(seg, __builtin_bit_cast(float, my_base + lane));
  lds_store<float>(work + 64 + 4 * (kWave * wv + lane), end);
  wg_barrier();
  float e[8];
  asm volatile(
      "ds_read_b32 %0, %8\n\tds_read_b32 %1, %8 offset:256\n\tds_read_b32 %2, %8 offset:512\n\t"
      "ds_read_b32 %3, %8 offset:768\n\tds_read_b32 %4, %8 offset:1024\n\tds_read_b32 %5, %8 offset:1280\n\t"
      "ds_read_b32 %6, %8 offset:1536\n\tds_read_b32 %7, %8 offset:1792\n\ts_waitcnt lgkmcnt(0)"
      : "=&v"(e[0]), "=&v"(e[1]), "=&v"(e[2]), "=&v"(e[3]), "=&v"(e[4]), "=&v"(e[5]), "=&v"(e[6]), "=&v"(e[7])
      : "v"(a_r + 4 * lane));
  float tot = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = __builtin_bit_cast(int, tot) - base[j];
    if (c >= 0 && c < kWave)
      tot = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e[j]), c));
    else
      tot = ordered_sum_continue<L>(a_sq + 4 * L * j, tot);
  }
  return tot;
}

// One Q8_0_ACT block from 32 lanes (an aligned group of 32 lanes, each holding
// element lane % 32): returns this lane's int8 and, in d, the block scale
// (amax / 127), as the engine's row quantiser.
// The group's amax: within each 16-lane row by DPP moves (quad swaps, row
// rotations), then across the group's two rows by one lane exchange; a max
// does not depend on the order (a lane whose own value is NaN keeps NaN, as
// with any order of strict greater-than steps). The whole group is active or
// inactive together.
__device__ inline int q8_lane_quant(float y, float& d) {
#pragma clang fp contract(off)
  float amax = fabsf(y);
  float o = dpp_mov<0xB1>(amax);  // quad_perm [1,0,3,2]
  amax = o > amax ? o : amax;
  o = dpp_mov<0x4E>(amax);  // quad_perm [2,3,0,1]
  amax = o > amax ? o : amax;
  o = dpp_mov<0x124>(amax);  // row_ror:4
  amax = o > amax ? o : amax;
  o = dpp_mov<0x128>(amax);  // row_ror:8
  amax = o > amax ? o : amax;
  o = __shfl_xor(amax, 16, 32);
  amax = o > amax ? o : amax;
  d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  int q = (int)__builtin_rintf(y * id);
  return q > 127 ? 127 : (q < -127 ? -127 : q);
}

}  // namespace mi
