// decode.hip -- fused ATTN_QK -> causal SOFTMAX -> ATTN_KQV for one query
// token (src/ops_cpu.cpp:304-410 with n_tokens == 1), HBM-bound, no MFMA.
//
// One launch, one kernel, no second pass.
//
// Work decomposition. A group is (item, KV head g, head chunk hc): the G <= 4*HS
// Q heads that read KV head g (GQA is an index mapping: every K/V row is read
// once for all G heads, never copied). Each group is served by kpg workgroups
// (the host sizes kpg so the launch has about one workgroup per CU). The
// group's positions are cut into sub-tiles of 16 (the last one partial) that
// the waves of its workgroups take one at a time:
//   - claims (groups long enough that each wave streams several ring
//     cycles): each wave's first NB sub-tiles are fixed (a prefix of the
//     group spread over its workgroups); every refill then claims one more
//     sub-tile from the group's counter in device memory. The claim is issued
//     a whole ring cycle before its result is used, so its latency hides
//     behind the loads in flight, and the workgroups of a group finish
//     together however unevenly the memory system serves them;
//   - local takes (short groups, where a claim's round trip would not hide):
//     part p of the group's kpg workgroups owns sub-tiles p, p + kpg,
//     p + 2 kpg, ..., and its waves take them in turn from an LDS counter.
//
// Streaming. Each wave owns an LDS ring of NB slots; a slot holds one
// sub-tile's K rows then its V rows, written by buffer_load ... lds (direct to
// LDS, no registers). Every slot is refilled once per ring cycle, with a
// zero-sized resource that reads nothing once the wave has run out of
// sub-tiles, so the number of memory operations issued after any slot's K (or
// V) is always the same and the waits are fixed vmcnt values. Rows past n_kv
// lie outside the sub-tile's bounded resource and arrive as zeros without a
// memory request. The 16-byte slots of each K row are stored XOR-swizzled by
// row, so the lane-per-row reads below are free of bank conflicts.
//
// Per sub-tile (lane = (row r = lane / 16, column i = lane % 16)):
//   QK  lane (position i, head slots r + 4h): the lane dots its K row with the
//       query, whose elements come from a DPP row broadcast (v_fmac_f32_dpp
//       row_newbcast) -- the queries stay spread over the 16 lanes of a row;
//   softmax in base 2, running max per head by DPP row reduction;
//   PV  lane (dims 4i + 64e .., head slots r + 4h): O += P.V with plain FMAs;
//       the 16 probabilities of a row go through a small per-wave LDS area and
//       come back as a broadcast read.
//
// Combining. At the end the waves' (m, l, acc) meet in LDS. With kpg == 1 the
// workgroup writes O. Otherwise partials are merged across workgroups with the
// stable rescaling O = sum_s 2^(m_s - M) A_s / sum_s 2^(m_s - M) L_s, in part
// order, by one of two protocols:
//   - early (groups of 2..kDecodeEarlyMax workgroups): every part counts
//     itself in the group's start counter when it starts (the result is read
//     only at the end, so the round trip hides behind the streaming); part 0
//     merges, the others store their record as 64-bit (value, launch epoch)
//     words and exit. The merger polls the records until every word carries
//     this launch's epoch and merges, so after the last part finishes only
//     that part's stores, one poll and the merge remain. The wait is bounded:
//     a merger that runs out of polls marks
//     the start counter. If every part had started by then, they are all
//     running and it keeps waiting; otherwise it stores its own record and
//     exits, and the parts that start after the mark (they see it in their
//     start count) count themselves again at their end: the last of them
//     merges. So a group whose parts cannot all be resident at once (other
//     work holds the CUs) costs time, never correctness, and the fallback is
//     counted in the workspace's status words;
//   - flat (larger groups whose launch fits the device at once): every part
//     counts itself as started, stores its record as stamped words and then
//     merges its own slice of the output (a range of (head, 4 dims) pairs)
//     over every part's record: R lanes (R the power of two >= kpg) poll one
//     pair's R records, a butterfly combines them in a fixed order, and one
//     lane writes the 4 outputs. One poll round after the last part's stores
//     instead of two arrival round trips and two record reads. Bounded like
//     the early merge: a part that runs out of polls marks the start counter;
//     if some part had not started by then it leaves its slice to the last
//     part to start (which sees the mark in its start count and merges every
//     slice), otherwise it keeps waiting;
//   - teams (larger groups otherwise): every workgroup stores its record, waits
//     for the stores and bumps its team's arrival counter; the last arriver of
//     a team merges the team's records, and the last team merges the team
//     results.
// Counters come in two sets: launch e uses set e & 1, which launch e - 1
// cleared, and clears set (e + 1) & 1 for launch e + 1, so no counter is ever
// re-armed by a merger that might run before a late increment.
#include <cstdlib>
#include <type_traits>

#include "attn_common.h"
#include "kernels.h"

namespace mi {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
// Cache policy of buffer accesses that must be coherent across the XCDs' L2
// caches (the encoding the compiler uses for agent-scope atomic loads/stores).
constexpr int kSc1 = 16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));


template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

__device__ inline float row_sum16(float x) {
  x += dpp_mov<0xB1>(x);
  x += dpp_mov<0x4E>(x);
  x += dpp_mov<0x141>(x);
  x += dpp_mov<0x140>(x);
  return x;
}

// ---------------------------------------------------------------------------
// DPP multiply-add blocks. v_fmac_f32_dpp with row_newbcast:J takes its first
// factor from lane J of each row of 16. The compiler does not form it (the
// accumulator is tied), so each block is one asm statement with a fixed
// order: no accumulator is written by two DPP instructions less than three
// instructions apart, and the first block of a chain initialises its
// accumulators with v_mul_f32_dpp inside the block. Inputs written by a VALU
// instruction (probabilities, rescaled accumulators, widened F16 elements) are
// separated from the block by an s_nop 1 (two wait states): NOP prefixes the
// block with it.
// ---------------------------------------------------------------------------
#define MI_DPP(op, d, q, k, j) #op "_dpp %" #d ", %" #q ", %" #k " row_newbcast:%" #j " row_mask:0xf bank_mask:0xf\n\t"
#define MI_NOP "s_nop 1\n\t"

// QK, four elements of one source lane J: s[h][e % (4/HS)] += bcast_J(q[h][e]) * k[e].
#define MI_QK2_FIRST                                                              \
  MI_DPP(v_mul_f32, 0, 4, 12, 16) MI_DPP(v_mul_f32, 2, 8, 12, 16)                 \
  MI_DPP(v_mul_f32, 1, 5, 13, 16) MI_DPP(v_mul_f32, 3, 9, 13, 16)                 \
  MI_DPP(v_fmac_f32, 0, 6, 14, 16) MI_DPP(v_fmac_f32, 2, 10, 14, 16)              \
  MI_DPP(v_fmac_f32, 1, 7, 15, 16) MI_DPP(v_fmac_f32, 3, 11, 15, 16)
#define MI_QK2_NEXT                                                               \
  MI_DPP(v_fmac_f32, 0, 4, 12, 16) MI_DPP(v_fmac_f32, 2, 8, 12, 16)               \
  MI_DPP(v_fmac_f32, 1, 5, 13, 16) MI_DPP(v_fmac_f32, 3, 9, 13, 16)               \
  MI_DPP(v_fmac_f32, 0, 6, 14, 16) MI_DPP(v_fmac_f32, 2, 10, 14, 16)              \
  MI_DPP(v_fmac_f32, 1, 7, 15, 16) MI_DPP(v_fmac_f32, 3, 11, 15, 16)
#define MI_QK2_IN                                                                 \
  "v"(q[0][0]), "v"(q[0][1]), "v"(q[0][2]), "v"(q[0][3]), "v"(q[1][0]), "v"(q[1][1]), \
      "v"(q[1][2]), "v"(q[1][3]), "v"(k[0]), "v"(k[1]), "v"(k[2]), "v"(k[3]), "i"(J)
#define MI_QK1_FIRST                                                              \
  MI_DPP(v_mul_f32, 0, 4, 8, 12) MI_DPP(v_mul_f32, 1, 5, 9, 12)                   \
  MI_DPP(v_mul_f32, 2, 6, 10, 12) MI_DPP(v_mul_f32, 3, 7, 11, 12)
#define MI_QK1_NEXT                                                               \
  MI_DPP(v_fmac_f32, 0, 4, 8, 12) MI_DPP(v_fmac_f32, 1, 5, 9, 12)                 \
  MI_DPP(v_fmac_f32, 2, 6, 10, 12) MI_DPP(v_fmac_f32, 3, 7, 11, 12)
#define MI_QK1_IN                                                                 \
  "v"(q[0][0]), "v"(q[0][1]), "v"(q[0][2]), "v"(q[0][3]), "v"(k[0]), "v"(k[1]), "v"(k[2]), \
      "v"(k[3]), "i"(J)

template <int J, bool FIRST, bool NOP>
__device__ __forceinline__ void qk4_2(float (&s)[2][2], const float (&q)[2][4], const float (&k)[4]) {
#define MI_OUT_W "=&v"(s[0][0]), "=&v"(s[0][1]), "=&v"(s[1][0]), "=&v"(s[1][1])
#define MI_OUT_RW "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[1][0]), "+v"(s[1][1])
  if constexpr (FIRST && NOP) asm(MI_NOP MI_QK2_FIRST : MI_OUT_W : MI_QK2_IN);
  else if constexpr (FIRST) asm(MI_QK2_FIRST : MI_OUT_W : MI_QK2_IN);
  else if constexpr (NOP) asm(MI_NOP MI_QK2_NEXT : MI_OUT_RW : MI_QK2_IN);
  else asm(MI_QK2_NEXT : MI_OUT_RW : MI_QK2_IN);
#undef MI_OUT_W
#undef MI_OUT_RW
}

template <int J, bool FIRST, bool NOP>
__device__ __forceinline__ void qk4_1(float (&s)[1][4], const float (&q)[1][4], const float (&k)[4]) {
#define MI_OUT_W "=&v"(s[0][0]), "=&v"(s[0][1]), "=&v"(s[0][2]), "=&v"(s[0][3])
#define MI_OUT_RW "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[0][2]), "+v"(s[0][3])
  if constexpr (FIRST && NOP) asm(MI_NOP MI_QK1_FIRST : MI_OUT_W : MI_QK1_IN);
  else if constexpr (FIRST) asm(MI_QK1_FIRST : MI_OUT_W : MI_QK1_IN);
  else if constexpr (NOP) asm(MI_NOP MI_QK1_NEXT : MI_OUT_RW : MI_QK1_IN);
  else asm(MI_QK1_NEXT : MI_OUT_RW : MI_QK1_IN);
#undef MI_OUT_W
#undef MI_OUT_RW
}

template <int J, int HS, bool FIRST, bool NOP>
__device__ __forceinline__ void qk4(float (&s)[HS][4 / HS], const float (&q)[HS][4], const float (&k)[4]) {
  if constexpr (HS == 2)
    qk4_2<J, FIRST, NOP>(s, q, k);
  else
    qk4_1<J, FIRST, NOP>(s, q, k);
}

#undef MI_QK2_FIRST
#undef MI_QK2_NEXT
#undef MI_QK2_IN
#undef MI_QK1_FIRST
#undef MI_QK1_NEXT
#undef MI_QK1_IN
#undef MI_PV2
#undef MI_PV1
#undef MI_NOP
#undef MI_DPP



// ---------------------------------------------------------------------------
// Matrix-core compute (the MF kernels). Per 16-position sub-tile a wave
// computes S^T (16 positions x 16 head columns) = K Q^T with 16x16x32 MFMAs
// and O^T (dims x 16 head columns) += V^T P with 16x16x16 MFMAs; lane l holds
// S^T[4 (l/16) + r][l % 16] (r < 4), which is exactly its B operand of the PV
// product, so the probabilities never leave the lane. With an F32 cache every
// F32 operand x is split as x = hi + lo (bf16, round to nearest) and a
// product a b is formed as ah bh + ah bl + al bh (the lo lo term is below
// 2^-16 of it); with an F16 cache the cache operands are exact in f16 and the
// F32 ones (Q, P) are split as f16 pairs. Products of bf16 or f16 numbers are
// exact in the FP32 accumulators.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

template <int N, typename V>
__device__ __forceinline__ void split_to(const float* x, V& hi, V& lo) {
  typedef decltype(hi[0] + hi[0]) E;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const E h = (E)x[i];
    hi[i] = h;
    lo[i] = (E)(x[i] - (float)h);
  }
}
__device__ __forceinline__ f32x4 mfma_k32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_k32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_k16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                   0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_k16(half4_t a, half4_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// V rows of the MF kernels: 16-byte slot j of row r is stored at slot
// j ^ swv(r), so the four row groups (r / 4) of one PV operand read (16
// consecutive elements of rows 4 g + i) fall in distinct banks.
template <int ELT>
__host__ __device__ constexpr int swv(int r) {
  return ((r >> 2) & 3) * ELT;
}

template <int D, typename KT, int HS, int NWV, bool DYN>
struct DecodeCfg {
  static constexpr int ELT = (int)sizeof(KT);
  static constexpr int RB = D * ELT;              // bytes per cache row
  static constexpr int NSLOT = RB / 16;           // 16-byte slots per row
  static constexpr int SE = 16 / ELT;             // elements per slot
  static constexpr int SUBB = kDecodeSub * RB;    // bytes of one K (or V) sub-tile
  static constexpr int NDK = SUBB / 1024;         // 1 KB loads per K (or V) sub-tile
  static constexpr int NDMA = 2 * NDK;
  static constexpr int OPS = NDMA + (DYN ? 1 : 0);  // vector memory operations per refill
  static constexpr int SLOTB = 2 * SUBB;          // ring slot: K rows, then V rows
  // 128 KB of ring per workgroup; 64 KB (two slots per wave) with an F16
  // cache at head_dim 128, measured 8% faster there than four slots (14.9 vs
  // 16.1 us per launch at n_kv 8192: its workgroups stream only 8 sub-tiles)
  static constexpr int RING = (D == 128 && ELT == 2 ? 64 : 128) * 1024;
  static constexpr int NB0 = RING / (NWV * SLOTB);
  static constexpr int NB = NB0 > 4 ? 4 : NB0;    // ring depth per wave
  static constexpr int HSL = 4 * HS;              // head slots (G <= HSL)
  static constexpr int DEPF = HSL * (D + 2);      // floats of one wave's deposit
  // A record: DEPF floats (team protocol) or DEPF 64-bit (value, epoch) words
  // (early protocol); every workgroup's record slot holds the larger.
  static constexpr int REC = 2 * DEPF;            // 4-byte units per record slot
  static constexpr int NP = HSL * D / 4;          // merge: (head slot, float4) pairs
  static constexpr int NSUB = NWV * kWave / NP;   // merge: record subsets
  static constexpr int NE = D / 64;               // float4 column blocks per lane
  // LDS layout (bytes). A wave's deposit overlays its own ring once the
  // wave's last loads have landed.
  static constexpr int L_RING = 0;
  static constexpr int L_P = L_RING + NWV * NB * SLOTB;  // per wave: P[head slot][16]
  static constexpr int L_FLAG = L_P + NWV * HSL * kDecodeSub * 4;
  static constexpr int L_TOTAL = L_FLAG + 16;
  static_assert(NB >= 2, "ring depth");
  static_assert(SUBB % 1024 == 0, "1 KB load granularity");
  static_assert(L_TOTAL <= 160 * 1024, "LDS budget");
  static_assert(DEPF * 4 <= NB * SLOTB, "a deposit fits its wave's ring");
  // After the loop: an early merger's own partial behind wave 0's deposit;
  // the merges' exchange area from wave 1's ring on.
  static constexpr int L_OWN = L_RING + ((DEPF * 4 + 15) & ~15);
  static constexpr int L_TMP = L_RING + NB * SLOTB;
  static_assert(L_OWN + NP * 24 <= L_RING + NB * SLOTB, "own partial in wave 0's ring");
  static_assert(NSUB <= 1 || L_TMP + NSUB * NP * 24 <= L_RING + NWV * NB * SLOTB, "merge exchange");
  // vmcnt allowed while waiting for a slot's K (its V and the later slots'
  // refills may still be in flight) and for its V. A refill issues its claim
  // (dynamic takes) before its loads.
  static constexpr int WAIT_K = NDK + OPS * (NB - 1);
  static constexpr int WAIT_V = OPS * (NB - 1);
  static_assert(WAIT_K <= 63, "vmcnt range");
  // Early protocol: teams of at most 32 (the counter block's team words).
  static constexpr int TEAM = NSUB * 8;
};

// One workgroup per CU at most is assumed only by the early protocol's
// bounded wait (it stays correct without it); the F16 head_dim-128 variant
// (64 KB ring) can share a CU. NWV / 4 waves per SIMD.
template <int D, typename KT, int HS, int NWV, bool DYN, bool MF>
__global__ __launch_bounds__(NWV* kWave) __attribute__((amdgpu_waves_per_eu(NWV / 4, NWV / 4)))
void decode_kernel(const DecodeParams p) {
  // Every scalar parameter and this grid row's item in one round of scalar
  // loads (the empty asm needs them all in registers at once; the compiler
  // would otherwise load each near its first use, in dependent rounds). Row y
  // of the grid serves item y, so the item's address needs no loaded value.
  const int ii = blockIdx.y;
  const DecodeItem& it = p.item[ii];
  const int a_n_rep = p.n_rep, a_n_head_kv = p.n_head_kv, a_n_chunks = p.n_chunks;
  const int a_gpi = p.gpi, a_n_wg = p.n_wg, a_early = p.early, a_det = p.det;
  const int a_max_polls = p.max_polls, a_ctr_groups = p.ctr_groups, a_clear_groups = p.clear_groups;
  const unsigned a_epoch = p.epoch;
  const float a_scale_log2e = p.scale_log2e;
  float* const a_rec = p.rec;
  unsigned* const a_cnt = p.cnt;
  unsigned* const a_status = p.status;
  const char* const it_k = it.k;
  const char* const it_v = it.v;
  const float* const it_q = it.q;
  float* const it_out = it.out;
  const int64_t k_s1 = it.k_s1, v_s1 = it.v_s1, q_s1 = it.q_s1, o_s1 = it.o_s1;
  const int n_kv = it.n_kv, kpg = it.kpg, wg0 = it.wg0;
  const int ks2 = (int)it.k_s2, vs2 = (int)it.v_s2;
  asm volatile("" ::"s"(a_n_rep), "s"(a_n_head_kv), "s"(a_n_chunks), "s"(a_gpi), "s"(a_n_wg), "s"(a_early), "s"(a_det),
               "s"(a_max_polls), "s"(a_ctr_groups), "s"(a_clear_groups), "s"(a_epoch), "s"(a_scale_log2e),
               "s"(a_rec), "s"(a_cnt), "s"(a_status), "s"(it_k), "s"(it_v), "s"(it_q), "s"(it_out), "s"(k_s1),
               "s"(v_s1), "s"(q_s1), "s"(o_s1), "s"(n_kv), "s"(kpg), "s"(wg0), "s"(ks2), "s"(vs2));
  typedef DecodeCfg<D, KT, HS, NWV, DYN> C;
  constexpr int HSL = C::HSL, NB = C::NB, NSLOT = C::NSLOT, NE = C::NE;
  constexpr int NACC = 4 / HS;
  constexpr bool F16 = C::ELT == 2;

  extern __shared__ __attribute__((aligned(16))) char lds_dyn[];
  lds_t* const lds = (lds_t*)lds_dyn;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;  // QK: position in the sub-tile; PV: column block
  const int hb = lane >> 4;   // head slots hb + 4 h

  // Records: one per workgroup, written and read with agent-coherent (sc1)
  // accesses through this resource (team protocol) or 64-bit atomics (early).
  const rsrc_t recr = make_rsrc(a_rec, (unsigned)(a_n_wg * C::REC * 4));

  // This launch's counter set; the groups the previous launch used in the
  // other set are cleared for the next launch (write-through stores: the next
  // launch's atomics are performed in memory), by every workgroup of the
  // grid, those past their row's item included.
  const size_t set_words = (size_t)a_ctr_groups * kCtrInts;
  unsigned* const cset = a_cnt + (size_t)(a_epoch & 1u) * set_words;
  {
    unsigned* const other = a_cnt + (size_t)((a_epoch + 1u) & 1u) * set_words;
    const int lin = blockIdx.y * gridDim.x + blockIdx.x, n_lin = gridDim.x * gridDim.y;
    for (int b = lin; b < a_clear_groups; b += n_lin)
      if (threadIdx.x < kCtrInts)
        __hip_atomic_store(other + (size_t)b * kCtrInts + threadIdx.x, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  // Rows are as wide as the launch's widest item.
  if ((int)blockIdx.x >= a_gpi * kpg) return;
  const int wg = wg0 + (int)blockIdx.x;  // this workgroup's record
  if (!DYN && !a_det) {  // (deterministic takes use no counter: no barrier to start)
    if (threadIdx.x == 0) lds_store<unsigned>(lds + C::L_FLAG + 4, 0u);  // LDS take counter
    wg_barrier();
  }
  const int local = wg - wg0;
  const int gl = local / kpg, part = local - gl * kpg;
  const int g = gl / a_n_chunks, hc = gl - g * a_n_chunks;
  // chunk hc: heads [hc n_rep / n_chunks, (hc + 1) n_rep / n_chunks) of the
  // KV head's n_rep (never empty, at most ceil(n_rep / n_chunks) heads)
  const int h_lo = hc * a_n_rep / a_n_chunks;
  const int head0 = g * a_n_rep + h_lo;
  const int G = (hc + 1) * a_n_rep / a_n_chunks - h_lo;
  const int gid = ii * a_gpi + gl;
  unsigned* const gcnt = cset + (size_t)gid * kCtrInts;
  const bool early = a_early && kpg > 1 && kpg <= kDecodeEarlyMax;
  const bool flat = a_early && kpg > kDecodeEarlyMax && kpg <= NWV * kWave;
  // Early protocol: count this part as started; the previous count (and the
  // merger's give-up mark, if it came first) is read at the end.
  unsigned started = 0u;
  if ((early || flat) && threadIdx.x == 0)
    started = __hip_atomic_fetch_add(gcnt + kCtrStarted, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // This lane's query elements for the DPP broadcast: qv[h][e][c] =
  // Q[head0 + hb + 4h][64e + 4col + c] (head slots past G repeat head G-1 and
  // are never written out). Requested before the first cache tile.
  float qv[HS][NE][4];
  if constexpr (!MF) {
    const char* q0 = reinterpret_cast<const char*>(it_q) + (int64_t)head0 * q_s1;
#pragma unroll
    for (int h = 0; h < HS; ++h)
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        const int hs = min(hb + 4 * h, G - 1);
        const f32x4 q4 = gload<f32x4>(q0 + (int64_t)hs * q_s1 + 4 * (64 * e + 4 * col));
        qv[h][e][0] = q4.x; qv[h][e][1] = q4.y; qv[h][e][2] = q4.z; qv[h][e][3] = q4.w;
      }
  }
  // MF: this lane's B operand of QK, Q[head hq][8 qg + 32 kk + i] (i < 8), as
  // hi/lo pairs; zero for head columns past G. With an F16 cache a head whose
  // largest |q| exceeds 2^14 is scaled by a power of two into the f16 range
  // (undone on its scores).
  constexpr int KK = D / 32, NT = D / 16;
  typedef typename std::conditional<F16, f16x8, bf16x8>::type op8_t;
  typedef typename std::conditional<F16, half4_t, bf16x4>::type op4_t;
  const int hq = lane & 15, qg = lane >> 4;
  float qf[KK][8];
  op8_t qh[KK], ql[KK];
  float sc_mf = a_scale_log2e;
  if constexpr (MF) {
    const char* q0 = reinterpret_cast<const char*>(it_q) + (int64_t)(head0 + min(hq, G - 1)) * q_s1;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        f32x4 q4 = gload<f32x4>(q0 + 4 * (8 * qg + 32 * kk + 4 * hh));
        if (hq >= G) q4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) qf[kk][4 * hh + c] = q4[c];
      }
  }

  // DMA lane offsets: load i of a sub-tile fills LDS bytes [1024 i, +1024).
  // K rows are swizzled (QK reads one row per lane); V rows are not (PV reads
  // one whole row per wave, which is conflict-free as it lies).
  unsigned offk[C::NDK], offv[C::NDK];
#pragma unroll
  for (int i = 0; i < C::NDK; ++i) {
    const int o = 1024 * i + 16 * lane;
    const int r = o / C::RB;
    const int j = ((o % C::RB) / 16) ^ swz<NSLOT>(r);
    offk[i] = (unsigned)(r * ks2 + 16 * j);
    offv[i] = MF ? (unsigned)(r * vs2 + 16 * (((o % C::RB) / 16) ^ swv<C::ELT>(r)))
                 : (unsigned)(r * vs2 + o % C::RB);
  }
  lds_t* const ring = lds + C::L_RING + wv * NB * C::SLOTB;
  // QK: logical slot j of this lane's row `col`.
  const lds_t* kp[NSLOT];
#pragma unroll
  for (int j = 0; j < NSLOT; ++j) kp[j] = ring + col * C::RB + 16 * (j ^ swz<NSLOT>(col));
  // PV: this lane's dims 4 col + 64 e of row r, rows RB apart in the slot.
  const lds_t* const vbase = ring + C::SUBB + 4 * col * C::ELT;
  lds_t* const pw = lds + C::L_P + wv * (HSL * kDecodeSub * 4);  // this wave's P area

  // Request stream over the group's sub-tiles [0, nsub) of 16 positions (the
  // last one partial: its rows past n_kv lie outside the sub-tile's bounded
  // resource and arrive as zeros without a memory request). rows[s]: first
  // position of the sub-tile in ring slot s, or -1 once the wave has run out.
  const int nsub = (n_kv + kDecodeSub - 1) / kDecodeSub;
  const rsrc_t none = make_rsrc(it_k, 0u);
  const char* const kg = it_k + (int64_t)g * k_s1;
  const char* const vg = it_v + (int64_t)g * v_s1;
  int rows[NB];
  bool drained = false;  // a refill past the share was skipped (wave-uniform)

  auto issue = [&](auto slc, int t) __attribute__((always_inline)) {
    constexpr int SL = decltype(slc)::value;
    lds_t* const slot = ring + SL * C::SLOTB;
    rsrc_t kr = none, vr = none;
    rows[SL] = -1;
    if (t < nsub) {
      const int r0 = kDecodeSub * t;
      const int nr = min(kDecodeSub, n_kv - r0);
      kr = make_rsrc(kg + (int64_t)r0 * ks2, (unsigned)((nr - 1) * ks2 + C::RB));
      vr = make_rsrc(vg + (int64_t)r0 * vs2, (unsigned)((nr - 1) * vs2 + C::RB));
      rows[SL] = r0;
    }
#pragma unroll
    for (int i = 0; i < C::NDK; ++i) dma16_nt(kr, slot + 1024 * i, offk[i]);
#pragma unroll
    for (int i = 0; i < C::NDK; ++i) dma16_nt(vr, slot + C::SUBB + 1024 * i, offv[i]);
  };
  // Dynamic takes: pend[s] is the claim (issued by lane 0 one ring cycle ago)
  // that names slot s's next sub-tile, nst + claim, after the fixed prefix of
  // nst = NB kpg NWV sub-tiles (wave wv of part `part` starts with sub-tile
  // (s kpg + part) NWV + wv in slot s). Claims of one slot are sequential, so
  // once a slot's claim runs past the group every later one does too.
  const int nst = NB * kpg * NWV;
  unsigned* const claim_ctr = gcnt + kCtrClaim;
  unsigned pend[NB];
  __attribute__((address_space(3))) unsigned* const take =
      reinterpret_cast<__attribute__((address_space(3))) unsigned*>(lds + C::L_FLAG + 4);
  // Local takes: the workgroup's t-th sub-tile is part + kpg t.
  // Deterministic launches: wave wv takes the workgroup's sub-tiles wv,
  // wv + NWV, ... in turn instead, so which wave accumulates which sub-tile,
  // and with it every rounding, is the same on every run.
  // In the vector-unit kernel with two waves per SIMD (NWV = 8), the second
  // wave of each SIMD (wv >= NWV / 2) takes only its first sub-tile and the
  // first waves take all the others, in turn: the issue arbiter favours the
  // older wave of a SIMD, and two waves issuing the vector products contend
  // for it. Measured on 24 layers x n_kv 4096: 23.25 us with equal shares,
  // 21.8 us this way (n_kv 32768: 134 -> 128 us); four waves per workgroup
  // with four ring slots each measured 24.4 us. The matrix-core kernel keeps
  // equal shares.
  constexpr bool SHIFT = !MF && NWV > 4;
  int seq = SHIFT ? 0 : wv;
  auto lds_take = [&]() __attribute__((always_inline)) {
    unsigned t = 0;
    if (a_det) {
      if constexpr (!SHIFT) {
        t = (unsigned)seq;
        seq += NWV;
      } else {
        const int k = seq++;
        if (k == 0)
          t = (unsigned)wv;
        else if (wv >= NWV / 2)
          t = (unsigned)nsub;  // none
        else
          t = (unsigned)(NWV + (k - 1) * (NWV / 2) + wv);
      }
    } else {
      if (lane == 0) t = __hip_atomic_fetch_add(take, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      t = (unsigned)__builtin_amdgcn_readfirstlane((int)t);
    }
    t = min(t, (unsigned)nsub);
    return (int)min((unsigned)part + (unsigned)kpg * t, (unsigned)nsub);
  };
  auto refill = [&](auto slc, bool first) __attribute__((always_inline)) {
    constexpr int SL = decltype(slc)::value;
    int t;
    if constexpr (DYN) {
      t = first ? (SL * kpg + part) * NWV + wv
                : (int)min((unsigned)nst + (unsigned)__builtin_amdgcn_readfirstlane((int)pend[SL]),
                           (unsigned)nsub);
      unsigned c = 0;
      if (lane == 0) c = __hip_atomic_fetch_add(claim_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      pend[SL] = c;
    } else {
      t = lds_take();
      if (drained) {  // nothing more for this wave (set by the first fill)
        rows[SL] = -1;
        return;
      }
    }
    issue(slc, t);
  };
  // The queries were requested first; they are in registers once at most the
  // ring's loads are outstanding (the empty asm makes the compiler wait here:
  // its wait counts the loads issued since, so every path below issues a
  // number of them known at compile time).
  auto q_ready = [&]() __attribute__((always_inline)) {
  if constexpr (!MF) {
#pragma unroll
    for (int h = 0; h < HS; ++h)
#pragma unroll
      for (int e = 0; e < NE; ++e)
        asm volatile("" : "+v"(qv[h][e][0]), "+v"(qv[h][e][1]), "+v"(qv[h][e][2]), "+v"(qv[h][e][3])::"memory");
  } else {
    // (the memory clobber keeps the compiler from hoisting the split, and
    // with it the wait for the queries, above the ring's loads)
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int i = 0; i < 8; i += 4)
        asm volatile("" : "+v"(qf[kk][i]), "+v"(qf[kk][i + 1]), "+v"(qf[kk][i + 2]), "+v"(qf[kk][i + 3])::"memory");
    if constexpr (F16) {
      float amax = 0.f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(qf[kk][i]));
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      if (amax > 16384.f) {  // 2^-e with 2^e >= amax / 2^14: exact scaling
        const int e = ilogbf(amax) - 13;
        const float f = ldexpf(1.f, -e);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
#pragma unroll
          for (int i = 0; i < 8; ++i) qf[kk][i] *= f;
        sc_mf = a_scale_log2e * ldexpf(1.f, e);
      }
    }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) split_to<8>(qf[kk], qh[kk], ql[kk]);
  }
  };
  // First fill: every slot (past the share through a zero-sized resource),
  // so that the loads after the queries' are a fixed count. In the vector
  // kernel (the short launches' choice), a wave whose share ends within it
  // issues no refill afterwards and from then on waits for all of its loads
  // instead of the fixed counts, which assume one refill per slot (measured:
  // -0.4 to -0.5 us on one-layer launches of 1 sub-tile per wave; a wave
  // that streams keeps issuing its empty refills to the end of its loop:
  // skipping them there, or in the matrix-core kernel, measured slower).
  static_for<0, NB>([&](auto slc) { refill(slc, true); });
  q_ready();
  if constexpr (!DYN && !MF) {
#pragma unroll
    for (int s2 = 0; s2 < NB; ++s2) drained |= rows[s2] < 0;
  }

  float m[HS], l[HS], acc[HS][NE][4];
  // MF: running max and this lane's partial sum for head column hq, and
  // O^T[16 nt + 4 qg + r][hq] in o[nt][r].
  float mf = -INFINITY, lf = 0.f;
  f32x4 o[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < HS; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < NE; ++e)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) acc[h][e][jj] = 0.f;
  }

  // MF: the sub-tile in ring slot SL on the matrix cores.
  auto process_mf = [&](auto slc) __attribute__((always_inline)) {
    constexpr int SL = decltype(slc)::value;
    const int row0 = rows[SL];
    constexpr int SOFF = SL * C::SLOTB;
    if (drained)
      wait_vmem<0>();
    else
      wait_vmem<C::WAIT_K>();
    // S^T = K Q^T: lane l's A operand is row hq of the sub-tile, elements
    // 8 qg + 32 kk + i. One accumulator per product term (independent MFMA
    // chains), summed in a fixed order.
    const lds_t* const krow = ring + SOFF + hq * C::RB;
    f32x4 s1 = {0.f, 0.f, 0.f, 0.f}, s2 = s1, s3 = s1;
    if constexpr (F16) {
      f16x8 kh[KK];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kh[kk] = lds_load<f16x8>(krow + 16 * ((qg + 4 * kk) ^ swz<NSLOT>(hq)));
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        s1 = mfma_k32(kh[kk], qh[kk], s1);
        s2 = mfma_k32(kh[kk], ql[kk], s2);
      }
    } else {
      bf16x8 kh[KK], kl[KK];
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const int c0 = 2 * qg + 8 * kk;
        const f32x4 a0 = lds_load<f32x4>(krow + 16 * (c0 ^ swz<NSLOT>(hq)));
        const f32x4 a1 = lds_load<f32x4>(krow + 16 * ((c0 + 1) ^ swz<NSLOT>(hq)));
        const float kf[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        split_to<8>(kf, kh[kk], kl[kk]);
      }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        s1 = mfma_k32(kh[kk], qh[kk], s1);
        s2 = mfma_k32(kh[kk], ql[kk], s2);
        s3 = mfma_k32(kl[kk], qh[kk], s3);
      }
    }

    // V^T operands (column 16 nt + hq of rows 4 qg + i for N-tile nt), read
    // while the QK products are in flight.
    if (!drained) wait_vmem<C::WAIT_V>();  // (drained: all landed above)
    const lds_t* const vb = ring + SOFF + C::SUBB;
    half4_t va[NT];
    bf16x4 vh[NT], vl[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if constexpr (F16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = 4 * qg + i, el = 16 * nt + hq;
          va[nt][i] = lds_load<_Float16>(vb + rr * C::RB + 16 * ((el / 8) ^ swv<2>(rr)) + 2 * (el % 8));
        }
      } else {
        float vf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = 4 * qg + i, el = 16 * nt + hq;
          vf[i] = lds_load<float>(vb + rr * C::RB + 16 * ((el / 4) ^ swv<4>(rr)) + 4 * (el % 4));
        }
        split_to<4>(vf, vh[nt], vl[nt]);
      }
    }

    // Online softmax (base 2) of head column hq over positions 4 qg + r.
    const f32x4 sacc = F16 ? s1 + s2 : (s1 + s2) + s3;
    float x[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = row0 + 4 * qg + r < n_kv ? sacc[r] * sc_mf : -INFINITY;
      mx = fmaxf(mx, x[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(mf, mx);
    const float alpha = fast_exp2(mf - mn);
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(x[r] - mn);
    lf = lf * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    mf = mn;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0ull) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt] *= alpha;
    }
    op4_t ph, pl;
    split_to<4>(pr, ph, pl);

    // O^T += V^T P.
    if constexpr (F16) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt] = mfma_k16(va[nt], ph, o[nt]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt] = mfma_k16(va[nt], pl, o[nt]);
    } else {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt] = mfma_k16(vh[nt], ph, o[nt]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt] = mfma_k16(vh[nt], pl, o[nt]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt] = mfma_k16(vl[nt], ph, o[nt]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot reads done before it is refilled
  };

  // The sub-tile in ring slot SL.
  auto process = [&](auto slc) __attribute__((always_inline)) {
    constexpr int SL = decltype(slc)::value;
    if constexpr (MF) {
      process_mf(slc);
      return;
    }
    const int row0 = rows[SL];
    constexpr int SOFF = SL * C::SLOTB;
    if (drained)
      wait_vmem<0>();
    else
      wait_vmem<C::WAIT_K>();

    // K slots are requested up to KW ahead of their multiply-adds (LDS reads
    // complete in order, so each block waits only for its own).
    typedef typename std::conditional<F16, f16x8, f32x4>::type kvec_t;
    constexpr int KW = NSLOT < 16 ? NSLOT : 16;
    kvec_t kk[NSLOT];
#pragma unroll
    for (int j = 0; j < KW; ++j) kk[j] = lds_load<kvec_t>(kp[j] + SOFF);
    float s[HS][NACC];
    static_for<0, NSLOT>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (j + KW < NSLOT) kk[j + KW] = lds_load<kvec_t>(kp[j + KW] + SOFF);
      if constexpr (!F16) {
        const float kf[4] = {kk[j].x, kk[j].y, kk[j].z, kk[j].w};
        float qs[HS][4];
#pragma unroll
        for (int h = 0; h < HS; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e) qs[h][e] = qv[h][j >> 4][e];
        qk4<j & 15, HS, j == 0, false>(s, qs, kf);
      } else {
        const float k0[4] = {(float)kk[j][0], (float)kk[j][1], (float)kk[j][2], (float)kk[j][3]};
        const float k1[4] = {(float)kk[j][4], (float)kk[j][5], (float)kk[j][6], (float)kk[j][7]};
        float q0[HS][4], q1[HS][4];
#pragma unroll
        for (int h = 0; h < HS; ++h)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            q0[h][e] = qv[h][(8 * j) >> 6][e];
            q1[h][e] = qv[h][(8 * j + 4) >> 6][e];
          }
        qk4<(2 * j) & 15, HS, j == 0, true>(s, q0, k0);
        qk4<(2 * j + 1) & 15, HS, false, true>(s, q1, k1);
      }
    });

    // Online softmax (base 2); the running max is uniform over a row.
    const bool valid = row0 + col < n_kv;
    float pr[HS];
#pragma unroll
    for (int h = 0; h < HS; ++h) {
      float x = s[h][0];
#pragma unroll
      for (int t = 1; t < NACC; ++t) x += s[h][t];
      x = valid ? x * a_scale_log2e : -INFINITY;
      const float mn = fmaxf(m[h], row_max16(x));
      const float alpha = fast_exp2(m[h] - mn);
      pr[h] = fast_exp2(x - mn);
      l[h] = l[h] * alpha + pr[h];
      m[h] = mn;
#pragma unroll
      for (int e = 0; e < NE; ++e)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[h][e][jj] *= alpha;
    }
    // P[head slot][position] to this wave's LDS area; read back, each row's
    // 16 probabilities broadcast to the 16 lanes of that row.
#pragma unroll
    for (int h = 0; h < HS; ++h) lds_store<float>(pw + 4 * ((hb + 4 * h) * kDecodeSub + col), pr[h]);
    wave_lds_fence();
    float pv[HS][kDecodeSub];
#pragma unroll
    for (int h = 0; h < HS; ++h)
#pragma unroll
      for (int q4 = 0; q4 < kDecodeSub / 4; ++q4) {
        const f32x4 t = lds_load<f32x4>(pw + 4 * ((hb + 4 * h) * kDecodeSub + 4 * q4));
        pv[h][4 * q4 + 0] = t.x; pv[h][4 * q4 + 1] = t.y; pv[h][4 * q4 + 2] = t.z; pv[h][4 * q4 + 3] = t.w;
      }

    if (!drained) wait_vmem<C::WAIT_V>();  // (drained: all landed above)
    typedef typename std::conditional<F16, half4_t, f32x4>::type vvec_t;
#pragma unroll
    for (int r = 0; r < kDecodeSub; ++r)
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        const vvec_t v4 = lds_load<vvec_t>(vbase + SOFF + r * C::RB + 64 * e * C::ELT);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int h = 0; h < HS; ++h) acc[h][e][jj] = fmaf(pv[h][r], (float)v4[jj], acc[h][e][jj]);
      }
    wave_lds_fence();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot reads done before it is refilled
  };

  // Ring slots in turn; a slot with a sub-tile is processed, every slot is
  // refilled; the loop ends once no slot holds a sub-tile.
  for (;;) {
    static_for<0, NB>([&](auto slc) {
      constexpr int SL = decltype(slc)::value;
      if (rows[SL] >= 0) process(slc);
      refill(slc, false);
    });
    bool any = false;
#pragma unroll
    for (int s = 0; s < NB; ++s) any |= rows[s] >= 0;
    if (!any) break;
  }

  // The waves meet in LDS: wave w's deposit at the start of its ring, once
  // its last loads (including the zero-filling ones) landed.
  wait_vmem<0>();
  unsigned* const flag = reinterpret_cast<unsigned*>(lds_dyn + C::L_FLAG);
  auto dep_at = [&](int w) { return reinterpret_cast<float*>(lds_dyn + C::L_RING + w * NB * C::SLOTB); };
  if constexpr (MF) {
    lf += __shfl_xor(lf, 16);
    lf += __shfl_xor(lf, 32);
    float* dw = dep_at(wv);
    if (hq < HSL) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) *reinterpret_cast<f32x4*>(dw + hq * D + 16 * nt + 4 * qg) = o[nt];
      if (qg == 0) {
        dw[HSL * D + 2 * hq] = mf;
        dw[HSL * D + 2 * hq + 1] = lf;
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < HS; ++h) l[h] = row_sum16(l[h]);
    float* dw = dep_at(wv);
#pragma unroll
    for (int h = 0; h < HS; ++h) {
#pragma unroll
      for (int e = 0; e < NE; ++e)
        *reinterpret_cast<f32x4*>(dw + (hb + 4 * h) * D + 64 * e + 4 * col) =
            f32x4{acc[h][e][0], acc[h][e][1], acc[h][e][2], acc[h][e][3]};
      if (col == 0) {
        dw[HSL * D + 2 * (hb + 4 * h)] = m[h];
        dw[HSL * D + 2 * (hb + 4 * h) + 1] = l[h];
      }
    }
  }
  wg_barrier();
  const bool merger = early && part == 0;
  float* const own = reinterpret_cast<float*>(lds_dyn + C::L_OWN);
  const unsigned long long ep = (unsigned long long)a_epoch << 32;
  constexpr unsigned long long kHi = 0xffffffff00000000ull;

  // Stamped record words of part q (early protocol): acc value c of pair
  // (hs, cq) at word hs (D + 2) + c D/4 + cq (consecutive lanes, whole
  // sectors), m at hs (D + 2) + D, l at + D + 1. 64-bit agent-scope atomics
  // keep each word whole: a reader that sees this launch's epoch in a word has
  // that word's value.
  auto rec_word = [&](int q, int hs, int k, int cq) __attribute__((always_inline)) {
    return reinterpret_cast<unsigned long long*>(a_rec) + (int64_t)(wg - part + q) * (C::REC / 2) +
           hs * (D + 2) + (k < 4 ? k * (D / 4) + cq : D + (k - 4));
  };
  auto store_stamped = [&](int hs, int cq, float mx, float lt, f32x4 at) __attribute__((always_inline)) {
    auto pk = [&](float v) { return ep | __builtin_bit_cast(unsigned, v); };
#pragma unroll
    for (int c = 0; c < 4; ++c)
      __hip_atomic_store(rec_word(part, hs, c, cq), pk(at[c]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (cq == 0) {
      __hip_atomic_store(rec_word(part, hs, 4, 0), pk(mx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(rec_word(part, hs, 5, 0), pk(lt), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  // Early merge: every part's partial in part order -- part `own_part`'s from
  // LDS (-1: none), the others' stamped records polled until their words carry
  // this launch's epoch, at most `polls` rounds. Subsets combined in order. On
  // success O is written and true returned; otherwise nothing is written.
  auto merge_early = [&](int own_part, int polls) __attribute__((always_inline)) -> bool {
    constexpr int NP = C::NP, NSUB = C::NSUB;
    constexpr int RB = (kDecodeEarlyMax + NSUB - 1) / NSUB;  // parts per subset
    wg_barrier();  // the own partial is in LDS
    const int tt = threadIdx.x;
    const int pair = tt % NP, sub = tt / NP;
    const int hs = pair / (D / 4), cq = pair % (D / 4);
    float mx = -INFINITY, lt = 0.f;
    f32x4 at = {0.f, 0.f, 0.f, 0.f};
    bool fresh = true;
    if (sub < NSUB) {
      auto polled = [&](int i) { return sub + i * NSUB < kpg && sub + i * NSUB != own_part; };
      auto word = [&](int i, int k) { return rec_word(min(sub + i * NSUB, kpg - 1), hs, k, cq); };
      unsigned long long w[RB][6];
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int k = 0; k < 6; ++k)
          w[i][k] = polled(i) ? __hip_atomic_load(word(i, k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ep;
      for (int n = 0;; ++n) {
        fresh = true;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int k = 0; k < 6; ++k) fresh &= (w[i][k] & kHi) == ep;
        if (fresh || n >= polls) break;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int k = 0; k < 6; ++k)
            if ((w[i][k] & kHi) != ep)
              w[i][k] = __hip_atomic_load(word(i, k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int q = sub + i * NSUB;
        if (q < kpg) {
          float v[6];
          if (q == own_part) {
            const float* e = own + pair * 6;
            v[0] = e[2]; v[1] = e[3]; v[2] = e[4]; v[3] = e[5]; v[4] = e[0]; v[5] = e[1];
          } else {
#pragma unroll
            for (int k = 0; k < 6; ++k) v[k] = __builtin_bit_cast(float, (unsigned)w[i][k]);
          }
          const float mn = fmaxf(mx, v[4]);
          const float wo = mx == -INFINITY ? 0.f : fast_exp2(mx - mn);
          const float wn = v[4] == -INFINITY ? 0.f : fast_exp2(v[4] - mn);
          lt = lt * wo + v[5] * wn;
          at = at * wo + f32x4{v[0], v[1], v[2], v[3]} * wn;
          mx = mn;
        }
      }
    }
    // every subset's thread agrees on freshness before anything is written
    flag[2] = 1u;
    wg_barrier();
    if (!fresh) flag[2] = 0u;
    wg_barrier();
    if (flag[2] == 0u) return false;
    if constexpr (NSUB > 1) {
      float* tmp = reinterpret_cast<float*>(lds_dyn + C::L_TMP);
      if (sub < NSUB) {
        tmp[(sub * NP + pair) * 6 + 0] = mx;
        tmp[(sub * NP + pair) * 6 + 1] = lt;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) tmp[(sub * NP + pair) * 6 + 2 + jj] = at[jj];
      }
      wg_barrier();
      if (sub == 0) {
#pragma unroll
        for (int s2 = 1; s2 < NSUB; ++s2) {
          const float* e = tmp + (s2 * NP + pair) * 6;
          const float mn = fmaxf(mx, e[0]);
          const float wo = mx == -INFINITY ? 0.f : fast_exp2(mx - mn);
          const float wn = e[0] == -INFINITY ? 0.f : fast_exp2(e[0] - mn);
          lt = lt * wo + e[1] * wn;
          at = at * wo + f32x4{e[2], e[3], e[4], e[5]} * wn;
          mx = mn;
        }
      }
    }
    if (sub == 0 && hs < G) {
      float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it_out) + (int64_t)(head0 + hs) * o_s1);
      gstore<f32x4>(o + 4 * cq, at * (1.f / lt));
    }
    return true;
  };
  // Thread 0's returning agent-scope atomic add, its result broadcast.
  auto atomic_bcast = [&](unsigned* c, unsigned inc) __attribute__((always_inline)) {
    wg_barrier();
    if (threadIdx.x == 0) flag[1] = __hip_atomic_fetch_add(c, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wg_barrier();
    return (unsigned)__builtin_amdgcn_readfirstlane((int)flag[1]);
  };
  // Combines (mo, lo, ao) into (m, l, a) with the stable rescaling.
  auto fold = [](float& m, float& l, f32x4& a, float mo, float lo, f32x4 ao) __attribute__((always_inline)) {
    const float mn = fmaxf(m, mo);
    const float wo = m == -INFINITY ? 0.f : fast_exp2(m - mn);
    const float wn = mo == -INFINITY ? 0.f : fast_exp2(mo - mn);
    l = l * wo + lo * wn;
    a = a * wo + ao * wn;
    m = mn;
  };

  // Flat protocol layout of the group's record area (64-bit (value, epoch)
  // words, kpg G (D + 2) of them): the npr = G D/4 pairs (pair = hs D/4 + cq)
  // form slices of FP pairs (FP the power of two >= npr / kpg, at most D/4, so
  // the slices tile the pairs exactly); acc value k of pair p of slice j from
  // part q at word ((4 j + k) kpg + q) FP + p, then m and l of head slot hs
  // from part q at 4 npr kpg + 2 (hs kpg + q) + {0, 1}. A part reading its
  // slice reads contiguous words.
  const int npr = G * (D / 4);
  int FP = 1;
  while (FP * kpg < npr) FP <<= 1;
  auto flat_word = [&](int idx) __attribute__((always_inline)) {
    return reinterpret_cast<unsigned long long*>(a_rec) + (int64_t)(wg - part) * (C::REC / 2) + idx;
  };
  auto store_flat = [&](int hs, int cq, float mx, float lt, f32x4 at) __attribute__((always_inline)) {
    auto pk = [&](float v) { return ep | __builtin_bit_cast(unsigned, v); };
    const int pi = hs * (D / 4) + cq, j = pi / FP, pp = pi % FP;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      __hip_atomic_store(flat_word(((4 * j + k) * kpg + part) * FP + pp), pk(at[k]), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (cq == 0) {
      const int w = 4 * npr * kpg + 2 * (hs * kpg + part);
      __hip_atomic_store(flat_word(w), pk(mx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(flat_word(w + 1), pk(lt), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  // Flat merge of slice j (pairs [j FP, (j + 1) FP)) over all kpg records, at
  // most `polls` poll rounds. In a round of PR pairs, lane t holds record
  // t / PR of pair t % PR (consecutive lanes read consecutive words); a
  // butterfly over the lanes of one pair combines a wave's records, and when a
  // pair's records span several waves their results meet in LDS, combined in
  // wave order. Every order is fixed, so the result does not depend on timing.
  // On success the slice's outputs are written and true returned; a failed
  // round writes none of its pairs.
  auto merge_flat = [&](int j, int polls) __attribute__((always_inline)) -> bool {
    constexpr int T = NWV * kWave;
    int R = 1;
    while (R < kpg) R <<= 1;
    const int PR = FP < T / R ? FP : T / R;   // pairs per round
    const int span = R * PR;                  // lanes of a round
    const int nw = span > kWave ? span / kWave : 1;  // waves a pair's records span
    const int t = (int)threadIdx.x;
    const int r = t / PR;
    for (int p0 = 0; p0 < FP; p0 += PR) {
      const int pp = p0 + t % PR, pi = j * FP + pp;
      const int hs = pi / (D / 4), cq = pi % (D / 4);
      const bool act = t < span && r < kpg;
      const int wml = 4 * npr * kpg + 2 * (hs * kpg + r);
      auto word = [&](int k) __attribute__((always_inline)) {
        return flat_word(k < 4 ? ((4 * j + k) * kpg + r) * FP + pp : wml + (k - 4));
      };
      unsigned long long w[6];
      bool fresh = true;
      if (act) {
#pragma unroll
        for (int k = 0; k < 6; ++k) w[k] = __hip_atomic_load(word(k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int n = 0;; ++n) {
          fresh = true;
#pragma unroll
          for (int k = 0; k < 6; ++k) fresh &= (w[k] & kHi) == ep;
          if (fresh || n >= polls) break;
#pragma unroll
          for (int k = 0; k < 6; ++k)
            if ((w[k] & kHi) != ep) w[k] = __hip_atomic_load(word(k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      flag[2] = 1u;
      wg_barrier();
      if (!fresh) flag[2] = 0u;
      wg_barrier();
      if (flag[2] == 0u) return false;
      float m = -INFINITY, l = 0.f;
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
      if (act) {
        a = f32x4{__builtin_bit_cast(float, (unsigned)w[0]), __builtin_bit_cast(float, (unsigned)w[1]),
                  __builtin_bit_cast(float, (unsigned)w[2]), __builtin_bit_cast(float, (unsigned)w[3])};
        m = __builtin_bit_cast(float, (unsigned)w[4]);
        l = __builtin_bit_cast(float, (unsigned)w[5]);
      }
      for (int x = PR; x < kWave && x < span; x <<= 1) {
        const float mo = __shfl_xor(m, x), lo = __shfl_xor(l, x);
        const f32x4 ao = {__shfl_xor(a[0], x), __shfl_xor(a[1], x), __shfl_xor(a[2], x), __shfl_xor(a[3], x)};
        fold(m, l, a, mo, lo, ao);
      }
      if (nw > 1) {
        float* tmp = reinterpret_cast<float*>(lds_dyn + C::L_TMP);
        const int wi = t / kWave;
        if (wi < nw && (t & (kWave - 1)) < PR) {
          float* e = tmp + ((t % PR) * nw + wi) * 6;
          e[0] = m; e[1] = l; e[2] = a[0]; e[3] = a[1]; e[4] = a[2]; e[5] = a[3];
        }
        wg_barrier();
        if (t < PR)
          for (int q = 1; q < nw; ++q) {
            const float* e = tmp + (t * nw + q) * 6;
            fold(m, l, a, e[0], e[1], f32x4{e[2], e[3], e[4], e[5]});
          }
        wg_barrier();
      }
      if (t < PR) {
        float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it_out) + (int64_t)(head0 + hs) * o_s1);
        gstore<f32x4>(o + 4 * cq, a * (1.f / l));
      }
    }
    return true;
  };
  // NaN outputs for slices [ja, jb) of a group whose records never arrived.
  auto lost_slices = [&](int ja, int jb) __attribute__((always_inline)) {
    for (int pi = ja * FP + (int)threadIdx.x; pi < jb * FP; pi += NWV * kWave) {
      const int hs = pi / (D / 4), cq = pi % (D / 4);
      float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it_out) + (int64_t)(head0 + hs) * o_s1);
      gstore<f32x4>(o + 4 * cq, f32x4{NAN, NAN, NAN, NAN});
    }
    if (threadIdx.x == 0) __hip_atomic_fetch_add(a_status + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  constexpr unsigned kGaveUp = 1u << 16;
  constexpr int kLongWait = 1 << 20;  // rounds; only a broken invariant exhausts it

  {
    // wave wv combines head slots wv + NWV t; lane = (slot t, float4 cq)
    constexpr int SPW = (HSL + NWV - 1) / NWV;  // head slots per wave
    const int t = lane / (D / 4), cq = lane % (D / 4);
    const int hs = wv + NWV * t;
    if (t < SPW && hs < HSL) {
      // every wave's (m, l) and float4 first (one round of LDS reads), then
      // the stable combine in wave order
      f32x2 mlw[NWV];
      f32x4 aw[NWV];
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const float* dw = dep_at(w);
        mlw[w] = *reinterpret_cast<const f32x2*>(dw + HSL * D + 2 * hs);
        aw[w] = *reinterpret_cast<const f32x4*>(dw + hs * D + 4 * cq);
      }
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < NWV; ++w) mx = fmaxf(mx, mlw[w].x);
      float lt = 0.f;
      f32x4 at = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const float wt = mlw[w].x == -INFINITY ? 0.f : fast_exp2(mlw[w].x - mx);  // a wave with no sub-tile
        lt += wt * mlw[w].y;
        at += wt * aw[w];
      }
      if (kpg == 1) {
        if (hs < G) {
          float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it_out) +
                                              (int64_t)(head0 + hs) * o_s1);
          gstore<f32x4>(o + 4 * cq, at * (1.f / lt));
        }
      } else if (merger) {
        float* e = own + (hs * (D / 4) + cq) * 6;
        e[0] = mx;
        e[1] = lt;
        *reinterpret_cast<f32x2*>(e + 2) = f32x2{at[0], at[1]};
        *reinterpret_cast<f32x2*>(e + 4) = f32x2{at[2], at[3]};
      } else if (flat) {
        if (hs < G) store_flat(hs, cq, mx, lt, at);
      } else if (early) {
        store_stamped(hs, cq, mx, lt, at);
      } else {
        const unsigned r0 = (unsigned)(wg * C::REC * 4);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, at), recr,
                                               r0 + 4 * (hs * D + 4 * cq), 0, kSc1);
        if (cq == 0)
          __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{mx, lt}), recr,
                                                r0 + 4 * (HSL * D + 2 * hs), 0, kSc1);
      }
    }
  }
  if (kpg == 1) return;
  if (flat) {
    // Part j < npr / FP merges slice j.
    const int n_slices = npr / FP;
    const bool mine = part < n_slices;
    if (threadIdx.x == 0) flag[3] = started;
    wg_barrier();
    const unsigned st = (unsigned)__builtin_amdgcn_readfirstlane((int)flag[3]);
    if (mine && !merge_flat(part, a_max_polls)) {
      // Out of polls: mark the start counter. If some part had not started,
      // leave this slice to the last part to start; otherwise every part is
      // running or done, and the records arrive.
      const unsigned g0 = atomic_bcast(gcnt + kCtrStarted, kGaveUp);
      if ((int)(g0 & (kGaveUp - 1)) < kpg) {
        if (threadIdx.x == 0) __hip_atomic_fetch_add(a_status + 0, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
      }
      if (!merge_flat(part, kLongWait)) lost_slices(part, part + 1);
    }
    // The last part to start, after some part gave up: every slice.
    if ((int)(st & (kGaveUp - 1)) == kpg - 1 && st >= kGaveUp)
      for (int j = 0; j < n_slices; ++j)
        if (!merge_flat(j, kLongWait)) lost_slices(j, j + 1);
    return;
  }
  if (early) {
    int own_part = part;
    if (!merger) {
      // The record is stored. Parts that started before any give-up mark
      // leave the merge to the merger (it keeps waiting for them); a part
      // that started after it counts itself among the late parts, and the
      // last of those merges.
      if (threadIdx.x == 0) flag[3] = started;
      wg_barrier();
      const unsigned st = (unsigned)__builtin_amdgcn_readfirstlane((int)flag[3]);
      if ((st & kGaveUp) == 0u) return;
      unsigned at = 0u;  // parts started before the mark, plus one (written by the merger)
      for (int n = 0; n < kLongWait && at == 0u; ++n)
        at = __hip_atomic_load(gcnt + kCtrGaveUpAt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int late = kpg - (int)(at - 1u);
      const unsigned d = atomic_bcast(gcnt + kCtrLate, 1u);
      if (at == 0u || (int)d != late - 1) return;
      own_part = -1;  // its own record is stored like the others
    } else if (!merge_early(part, a_max_polls)) {
      // Out of polls: mark the start counter. If every part had started, all
      // are running: keep waiting. Otherwise store this part's partial as a
      // stamped record, publish the give-up point and leave the merge to the
      // last late part.
      const unsigned g0 = atomic_bcast(gcnt + kCtrStarted, kGaveUp);
      if ((int)(g0 & (kGaveUp - 1)) < kpg) {
        constexpr int NP = C::NP;
        for (int pr = threadIdx.x; pr < NP; pr += NWV * kWave) {
          const float* e = own + pr * 6;
          store_stamped(pr / (D / 4), pr % (D / 4), e[0], e[1], f32x4{e[2], e[3], e[4], e[5]});
        }
        wait_vmem<0>();
        if (threadIdx.x == 0) {
          __hip_atomic_store(gcnt + kCtrGaveUpAt, (g0 & (kGaveUp - 1)) + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_fetch_add(a_status + 0, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
      }
    } else {
      return;
    }
    // Every part of the group is running or done: merge all partials (from
    // LDS for own_part, the rest from their records). The bound only guards
    // against a broken invariant (then the output is NaN and the group is
    // counted as lost).
    if (!merge_early(own_part, kLongWait)) {
      constexpr int NP = C::NP;
      for (int pr = threadIdx.x; pr < NP; pr += NWV * kWave) {
        const int hs = pr / (D / 4), cq = pr % (D / 4);
        if (hs < G) {
          float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it_out) + (int64_t)(head0 + hs) * o_s1);
          gstore<f32x4>(o + 4 * cq, f32x4{NAN, NAN, NAN, NAN});
        }
      }
      if (threadIdx.x == 0) __hip_atomic_fetch_add(a_status + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  wait_vmem<0>();  // the record stores have completed

  // Team protocol. The group's workgroups form teams of up to TEAM (as many
  // records as one merge round below reads). The last workgroup to arrive in
  // a team merges the team's records; with one team it writes O, otherwise it
  // stores the result as the record of the team's first part and the last
  // team to arrive merges the team records and writes O.
  constexpr int NP = C::NP, NSUB = C::NSUB;
  static_assert(NSUB >= 1, "one pair per thread");
  constexpr int RB8 = 8;                      // records per subset requested at once
  constexpr int TEAM = C::TEAM;               // records one round reads
  const int n_teams = (kpg + TEAM - 1) / TEAM;
  const int team = part / TEAM, team_first = team * TEAM;
  const int team_n = min(TEAM, kpg - team_first);
  // arrive at counter c, expecting n arrivals: true for the last one
  auto arrive = [&](unsigned* c, int n) __attribute__((always_inline)) {
    wg_barrier();
    if (threadIdx.x == 0) {
      const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      flag[0] = old == (unsigned)(n - 1) ? 1u : 0u;
    }
    wg_barrier();
    return __builtin_amdgcn_readfirstlane(flag[0]) != 0;
  };
  if (!arrive(gcnt + kCtrTeams + team, team_n)) return;

  const int tt = threadIdx.x;
  const int pair = tt % NP, sub = tt / NP;
  const int hs = pair / (D / 4), cq = pair % (D / 4);
  const unsigned rec0 = (unsigned)((wg - part) * C::REC * 4);  // the group's first record (bytes)
  // Stable merge of the records first, first + stride, ... (count of them);
  // subset 0 ends with the result.
  auto merge = [&](int first, int count, int stride, float& mx, float& lt, f32x4& at)
                   __attribute__((always_inline)) {
    mx = -INFINITY;
    lt = 0.f;
    at = f32x4{0.f, 0.f, 0.f, 0.f};
    if (sub < NSUB) {
      for (int r0 = sub; r0 < count; r0 += RB8 * NSUB) {
        float mr[RB8], lr[RB8];
        f32x4 ar[RB8];
#pragma unroll
        for (int i = 0; i < RB8; ++i) {  // clamped indices: every load is issued, extras weigh 0
          const unsigned rb = rec0 + (unsigned)((first + min(r0 + i * NSUB, count - 1) * stride) * C::REC * 4);
          const f32x2 ml = __builtin_bit_cast(
              f32x2, __builtin_amdgcn_raw_buffer_load_b64(recr, rb + 4 * (HSL * D + 2 * hs), 0, kSc1));
          mr[i] = ml.x;
          lr[i] = ml.y;
          ar[i] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(recr, rb + 4 * (hs * D + 4 * cq), 0, kSc1));
        }
#pragma unroll
        for (int i = 0; i < RB8; ++i) {
          const float mi = r0 + i * NSUB < count ? mr[i] : -INFINITY;
          const float mn = fmaxf(mx, mi);
          const float wo = mx == -INFINITY ? 0.f : fast_exp2(mx - mn);
          const float wn = mi == -INFINITY ? 0.f : fast_exp2(mi - mn);
          lt = lt * wo + lr[i] * wn;
          at = at * wo + ar[i] * wn;
          mx = mn;
        }
      }
    }
    if constexpr (NSUB > 1) {
      float* tmp = reinterpret_cast<float*>(lds_dyn + C::L_RING);  // the ring is drained
      if (sub < NSUB) {
        tmp[(sub * NP + pair) * 6 + 0] = mx;
        tmp[(sub * NP + pair) * 6 + 1] = lt;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) tmp[(sub * NP + pair) * 6 + 2 + jj] = at[jj];
      }
      wg_barrier();
      if (sub == 0) {
#pragma unroll
        for (int s2 = 1; s2 < NSUB; ++s2) {
          const float* e = tmp + (s2 * NP + pair) * 6;
          const float mn = fmaxf(mx, e[0]);
          const float wo = mx == -INFINITY ? 0.f : fast_exp2(mx - mn);
          const float wn = e[0] == -INFINITY ? 0.f : fast_exp2(e[0] - mn);
          lt = lt * wo + e[1] * wn;
          at = at * wo + f32x4{e[2], e[3], e[4], e[5]} * wn;
          mx = mn;
        }
      }
    }
  };
  auto write_out = [&](float lt, f32x4 at) __attribute__((always_inline)) {
    if (sub == 0 && hs < G) {
      float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it_out) + (int64_t)(head0 + hs) * o_s1);
      gstore<f32x4>(o + 4 * cq, at * (1.f / lt));
    }
  };

  float mx, lt;
  f32x4 at;
  merge(team_first, team_n, 1, mx, lt, at);
  if (n_teams == 1) {
    write_out(lt, at);
    return;
  }
  // the team's result replaces the record of its first part (all read above)
  if (sub == 0) {
    const unsigned r0 = rec0 + (unsigned)(team_first * C::REC * 4);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, at), recr, r0 + 4 * (hs * D + 4 * cq), 0, kSc1);
    if (cq == 0)
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, f32x2{mx, lt}), recr,
                                            r0 + 4 * (HSL * D + 2 * hs), 0, kSc1);
  }
  wait_vmem<0>();
  if (!arrive(gcnt + kCtrElect, n_teams)) return;
  merge(0, n_teams, TEAM, mx, lt, at);
  write_out(lt, at);
}

// Waves per workgroup: two per SIMD at head_dim 64 (a 128 KB ring still gives
// every wave two slots), one per SIMD at head_dim 128 (eight waves measured no
// faster there with an F16 cache: those launches are bound by latency).
template <int D, typename KT>
constexpr int decode_waves() {
  return D == 64 ? 8 : 4;
}

template <int D, typename KT, int HS, bool DYN, bool MF>
static hipError_t launch_decode_t(const DecodeParams& p, int grid_x, int n_items, hipStream_t stream) {
  constexpr int NWV = decode_waves<D, KT>();
  typedef DecodeCfg<D, KT, HS, NWV, DYN> C;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_kernel<D, KT, HS, NWV, DYN, MF>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, C::L_TOTAL);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL((decode_kernel<D, KT, HS, NWV, DYN, MF>), dim3((unsigned)grid_x, (unsigned)n_items),
                     dim3(NWV * kWave), C::L_TOTAL, stream, p);
  return hipGetLastError();
}

template <int D, typename KT, bool MF>
static hipError_t launch_decode_m(const DecodeParams& p, int grid_x, int n_items, int group, bool dyn,
                                  hipStream_t stream) {
  if (group > 4)
    return dyn ? launch_decode_t<D, KT, 2, true, MF>(p, grid_x, n_items, stream)
               : launch_decode_t<D, KT, 2, false, MF>(p, grid_x, n_items, stream);
  return dyn ? launch_decode_t<D, KT, 1, true, MF>(p, grid_x, n_items, stream)
             : launch_decode_t<D, KT, 1, false, MF>(p, grid_x, n_items, stream);
}

template <int D, typename KT>
static hipError_t launch_decode_h(const DecodeParams& p, int grid_x, int n_items, int group, bool dyn, bool mf,
                                  hipStream_t stream) {
  return mf ? launch_decode_m<D, KT, true>(p, grid_x, n_items, group, dyn, stream)
            : launch_decode_m<D, KT, false>(p, grid_x, n_items, group, dyn, stream);
}

int decode_wg_waves(int head_dim, bool f16) {
  (void)f16;
  return head_dim == 64 ? 8 : 4;
}

int decode_ring_slots(int head_dim, bool f16) {
  const int rb = head_dim * (f16 ? 2 : 4);
  const int ring = (head_dim == 128 && f16 ? 64 : 128) * 1024;
  const int nb = ring / (decode_wg_waves(head_dim, f16) * 2 * kDecodeSub * rb);
  return nb > 4 ? 4 : nb;
}

// Records one merge round reads (the team size of the cross-workgroup combine).
int decode_team(int head_dim, bool f16, int group) {
  const int hsl = group > 4 ? 8 : 4;
  const int threads = decode_wg_waves(head_dim, f16) * kWave;
  return threads / (hsl * head_dim / 4) * 8;
}

// A KV head's n_rep Q heads go in as few chunks of at most 8 as there can be
// (each chunk's workgroups read the KV head's rows once), cut as evenly as
// the kernels cut them: chunk hc holds heads [hc n_rep / c, (hc + 1) n_rep / c).
int decode_chunks(int n_rep) { return (n_rep + 7) / 8; }

int decode_group_size(int n_rep) {
  const int c = decode_chunks(n_rep);
  return (n_rep + c - 1) / c;
}

size_t decode_record_floats(int head_dim, int group) {
  const int hsl = group > 4 ? 8 : 4;
  return (size_t)(2 * hsl * (head_dim + 2));  // room for the early protocol's 64-bit words
}

hipError_t launch_decode(const DecodeParams& p, int grid_x, int n_items, int head_dim, bool f16, int group,
                         bool dyn, bool mf, hipStream_t stream) {
  if (grid_x < 1 || n_items < 1 || n_items > kDecodeMaxItems) return hipErrorInvalidValue;
  if (head_dim == 64)
    return f16 ? launch_decode_h<64, _Float16>(p, grid_x, n_items, group, dyn, mf, stream)
               : launch_decode_h<64, float>(p, grid_x, n_items, group, dyn, mf, stream);
  if (head_dim == 128)
    return f16 ? launch_decode_h<128, _Float16>(p, grid_x, n_items, group, dyn, mf, stream)
               : launch_decode_h<128, float>(p, grid_x, n_items, group, dyn, mf, stream);
  return hipErrorInvalidValue;
}

// Sets n words at p to v (workspace resets; a kernel rather than a memset so
// that it may be recorded in a graph).
__global__ __launch_bounds__(256) void fill_u32_kernel(unsigned* p, size_t n, unsigned v) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = v;
}

hipError_t launch_fill_u32(unsigned* p, size_t n, unsigned v, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, stream, p, n, v);
  return hipGetLastError();
}

}  // namespace mi
