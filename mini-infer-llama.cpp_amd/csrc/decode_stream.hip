// decode_stream.hip -- fused ATTN_QK -> causal SOFTMAX -> ATTN_KQV for one
// query token (src/ops_cpu.cpp:304-410 with n_tokens == 1) for launches whose
// groups each span several workgroups: HBM-bound, float products on the
// vector units (no MFMA), K/V straight into registers, and a merge by the last
// part of each group to arrive.
//
// Work decomposition. A group is (item, KV head g, head chunk hc): the Gc <= G
// Q heads that read KV head g (GQA is an index mapping: every K/V row is read
// once for all of them). Part p of the group's kpg workgroups owns the
// contiguous positions [n_kv p / kpg, n_kv (p + 1) / kpg); its NW waves take
// the part's 16-position sub-tiles w, w + NW, w + 2 NW, ... (a fixed
// assignment: the same bits on every run).
//
// Lane layout (lane = 16 kq + t): t is a position of the sub-tile, kq a block
// of 16 dims (dims 64 e + 16 kq + m, e < E = head_dim / 64).
//   loads  K: lane (kq, t) loads its 16 E elements of row t (bounded buffer
//          loads: rows past the part's end, and past n_kv, read as zero
//          without a request). V: lane (kq, t) loads element 64 e + 16 kq + t
//          of each of the 16 rows (one 64-lane load per row and e: a whole
//          row, coalesced). U sub-tiles per wave are in flight; every refill is
//          issued (an empty one through a zero-sized resource), so the waits
//          are fixed counts.
//   QK     s[h] += K[t][16 kq + m] * q[h][16 kq + m] for m < 16, the query
//          element from lane (kq, m) by a DPP row broadcast (v_fmac_f32_dpp
//          row_newbcast); then the four row partials are summed across rows
//          with the gfx950 lane swaps (v_permlane16/32_swap), so every row
//          holds the whole dot products of its 16 positions.
//   softmax  base 2 (the query is pre-scaled by scale * log2 e) against a
//          per-head reference m[h] that changes only when a score exceeds it:
//          then m[h] becomes the sub-tile's maximum plus kSlack and the
//          running sums are rescaled. So p = 2^(x - m) <= 1 always, and with
//          ordinary scores the reference is set once by the first sub-tile.
//   PV     o[h][e] (lane (kq, t) owns dim 64 e + 16 kq + t of every head) +=
//          p[t'][h] * V[t'][64 e + 16 kq + t] over the 16 rows t', the
//          probability from lane (kq, t') by a DPP row broadcast.
//
// Combining. The waves' (m, l, o) meet in LDS and are merged in wave order.
// With kpg == 1 the workgroup writes O. Otherwise every part stores its
// record as 64-bit (value, launch stamp) words and takes a ticket from the
// group's arrival counter (taken when its streaming ends, so its round trip
// hides behind the combine); the part holding the last ticket merges: it
// polls the other parts' records until every word carries this launch's
// stamp and merges all parts in part order (O = sum_p 2^(m_p - M) A_p /
// sum_p 2^(m_p - M) L_p, the same bits whichever part merges). Every other
// part has already taken its ticket, so it is running and its record will
// arrive: the wait needs no co-residency. It is bounded all the same (a group
// whose records never arrive is written as NaN and counted as lost).
// Counters follow the workspace's two-set protocol: launch e uses set e & 1
// (zero on entry) and clears set (e + 1) & 1 for launch e + 1.
#include <type_traits>

#include "attn_common.h"
#include "kernels.h"

namespace mi {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr float kSlack = 8.0f;  // a new reference sits this far (log2) above the sub-tile's maximum

template <int I, int N, typename F>
__device__ __forceinline__ void sfor(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    sfor<I + 1, N>(f);
  }
}

// The sum of x over the four rows of 16 lanes, in every lane (the same bits in
// every lane: each step adds the same two values in every lane of a pair).
// v_permlane16_swap exchanges the odd rows of its first operand with the even
// rows of its second; v_permlane32_swap the upper half of the first with the
// lower half of the second. Written as asm (the s_nop gives the two wait
// states a VALU write of an operand needs before the swap reads it).
__device__ inline float rows_sum4(float x) {
  float y = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  float a = x + y;
  float b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}

// acc + bcast_J(q) * k and bcast_J(q) * k (lane J of each row of 16 supplies
// q), one instruction each. Volatile, so they keep their program order: the
// callers interleave accumulators so that no accumulator is written by a DPP
// instruction fewer than two wait states before the next DPP instruction
// reads it, and pin every other VGPR operand written by the VALU behind an
// s_nop 1 (the conservative reading of the DPP read-after-VALU-write rule:
// every VGPR operand of a DPP instruction counts).
template <int J>
__device__ inline void fmac_b(float& acc, float q, float k) {
  asm volatile("v_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
               : "+v"(acc)
               : "v"(q), "v"(k), "i"(J));
}
template <int J>
__device__ inline void mul_b(float& acc, float q, float k) {
  asm volatile("v_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf"
               : "=v"(acc)
               : "v"(q), "v"(k), "i"(J));
}

// Orders every earlier VALU write of the 16 values before the next DPP
// instruction with two wait states between (the s_nop); NOP = false only
// orders them (a later pin supplies the wait states).
template <bool NOP>
__device__ inline void pin16(float* v) {
  if constexpr (NOP)
    asm volatile("s_nop 1"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),
                   "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]),
                   "+v"(v[14]), "+v"(v[15])::"memory");
  else
    asm volatile(""
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),
                   "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]), "+v"(v[12]), "+v"(v[13]),
                   "+v"(v[14]), "+v"(v[15])::"memory");
}

__device__ inline float row_sum16s(float x) {
  x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_mov<0x141>(x);  // row_half_mirror
  x += dpp_mov<0x140>(x);  // row_mirror
  return x;
}

template <typename KT>
struct Elt;
template <>
struct Elt<float> {
  // K: 16 floats per (lane, e) = four 16-byte loads; V: one float per load
  static constexpr int NK4 = 4;
};
template <>
struct Elt<_Float16> {
  static constexpr int NK4 = 2;
};

}  // namespace

template <int E, typename KT, int G, int NW, int U>
__global__ __launch_bounds__(NW* kWave) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
void stream_decode_kernel(const DecodeParams p) {
  constexpr int D = 64 * E;
  constexpr int ELT = (int)sizeof(KT);
  constexpr int RB = D * ELT;
  constexpr int NK4 = Elt<KT>::NK4;
  constexpr bool F16 = ELT == 2;
  constexpr int NT = NW * kWave;

  const int ii = blockIdx.y;
  const DecodeItem& it = p.item[ii];
  const int n_rep = p.n_rep, n_chunks = p.n_chunks, gpi = p.gpi;
  const unsigned epoch = p.epoch;
  const int n_kv = it.n_kv, kpg = it.kpg;
  const int ks2 = (int)it.k_s2, vs2 = (int)it.v_s2;

  // This launch's counter set; the other set's groups [0, clear_groups) are
  // cleared for the next launch by the whole grid.
  const size_t set_words = (size_t)p.ctr_groups * kCtrInts;
  unsigned* const cset = p.cnt + (size_t)(epoch & 1u) * set_words;
  {
    unsigned* const other = p.cnt + (size_t)((epoch + 1u) & 1u) * set_words;
    const int lin = blockIdx.y * gridDim.x + blockIdx.x, n_lin = gridDim.x * gridDim.y;
    for (int b = lin; b < p.clear_groups; b += n_lin)
      if (threadIdx.x < kCtrInts)
        __hip_atomic_store(other + (size_t)b * kCtrInts + threadIdx.x, 0u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  if ((int)blockIdx.x >= gpi * kpg) return;  // rows are as wide as the widest item

  __shared__ float wm[NW][G], wl[NW][G];
  __shared__ float wo[NW][G][D];
  __shared__ unsigned merge_flag;

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = lane & 15, kq = lane >> 4;

  const int local = blockIdx.x;
  const int gl = local / kpg, part = local - gl * kpg;
  const int g = gl / n_chunks, hc = gl - g * n_chunks;
  const int h_lo = hc * n_rep / n_chunks;
  const int head0 = g * n_rep + h_lo;
  const int Gc = (hc + 1) * n_rep / n_chunks - h_lo;  // heads of this chunk (<= G)
  const int gid = ii * gpi + gl;
  const int wg = it.wg0 + local;

  // The query, pre-scaled into base-2 logits: qd[h][e] = q[head0 + h][64 e +
  // 16 kq + t] * scale * log2 e (head slots past Gc repeat the last head; their
  // results are never written).
  float qd[G][E];
  {
    const char* q0 = reinterpret_cast<const char*>(it.q);
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < E; ++e)
        qd[h][e] = gload<float>(q0 + (int64_t)(head0 + min(h, Gc - 1)) * it.q_s1 + 4 * (64 * e + 16 * kq + t)) *
                   p.scale_log2e;
  }

  // The part's positions and this wave's sub-tiles.
  const int P0 = (int)((int64_t)n_kv * part / kpg), P1 = (int)((int64_t)n_kv * (part + 1) / kpg);
  const int ns = (P1 - P0 + kDecodeSub - 1) / kDecodeSub;
  const int mine = w < ns ? (ns - w + NW - 1) / NW : 0;
  const char* const kg = it.k + (int64_t)g * it.k_s1;
  const char* const vg = it.v + (int64_t)g * it.v_s1;

  // Per-lane load offsets within a sub-tile (range-checked: K rows past the
  // sub-tile's valid rows read as zero). V rows come through the scalar
  // offset, clamped to the last valid row (finite data whose probability is
  // zero), so no V load reaches past n_kv.
  unsigned koff[E][NK4];
#pragma unroll
  for (int e = 0; e < E; ++e)
#pragma unroll
    for (int j = 0; j < NK4; ++j) koff[e][j] = (unsigned)(t * ks2 + (64 * e + 16 * kq) * ELT + 16 * j);
  unsigned voff[E];
#pragma unroll
  for (int e = 0; e < E; ++e) voff[e] = (unsigned)((64 * e + 16 * kq + t) * ELT);

  // (the 16 loaded bytes are reinterpreted as a whole as floats or halves:
  // ROCm 7.2 clang folds every element of an unsigned 4-vector from
  // raw_buffer_load_b128 that is bit-cast to float separately to element 0)
  f32x4 kb[U][E][NK4];
  unsigned vb[U][E][kDecodeSub];
  int nrs[U];  // valid rows of the sub-tile in each slot (0: none)

  auto issue = [&](auto uc, int s) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    const int r0 = P0 + kDecodeSub * s;
    const int nr = s < ns ? min(kDecodeSub, P1 - r0) : 0;
    nrs[u] = nr;
    const rsrc_t kr = make_rsrc(kg + (int64_t)(nr > 0 ? r0 : 0) * ks2, nr > 0 ? (unsigned)((nr - 1) * ks2 + RB) : 0u);
    const rsrc_t vr = make_rsrc(vg + (int64_t)(nr > 0 ? r0 : 0) * vs2, nr > 0 ? (unsigned)((nr - 1) * vs2 + RB) : 0u);
#pragma unroll
    for (int e = 0; e < E; ++e)
#pragma unroll
      for (int j = 0; j < NK4; ++j)
        kb[u][e][j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, koff[e][j], 0, 0));
    // Default cache policy for K and V here: with this kernel's access
    // pattern (per-lane 16-byte K pieces, narrow per-row V loads that share
    // cache lines) nontemporal loads cost 5 us on 24 layers x n_kv 4096.
    const int last = nr > 0 ? nr - 1 : 0;
#pragma unroll
    for (int r = 0; r < kDecodeSub; ++r) {
      const int so = min(r, last) * vs2;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if constexpr (F16)
          vb[u][e][r] = (unsigned)__builtin_amdgcn_raw_buffer_load_b16(vr, voff[e], so, 0);
        else
          vb[u][e][r] = __builtin_amdgcn_raw_buffer_load_b32(vr, voff[e], so, 0);
      }
    }
  };

  // Running state: reference m[h] (wave-uniform), this lane's sum of p over
  // its position slot, and its output dims in NPV partial accumulators (more
  // than one only for few heads, so that consecutive DPP multiply-adds never
  // write the same accumulator back to back).
  constexpr int NPQ = G >= 3 ? 1 : (G == 2 ? 2 : 3);          // QK partials per head
  constexpr int NPV = G * E >= 3 ? 1 : (G * E == 2 ? 2 : 3);  // PV partials per (head, e)
  // slot-padded register groups for the pins (16 values each)
  constexpr int NPIN_O = (G * E * NPV + 15) / 16;
  float m[G], l[G];
  float ob[NPIN_O * 16];
#pragma unroll
  for (int i = 0; i < NPIN_O * 16; ++i) ob[i] = 0.f;
  auto O = [&](int h, int e, int pp) -> float& { return ob[(h * E + e) * NPV + pp]; };
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
  }

  // The first ring of loads, then the query pinned after its scaling (two
  // wait states before its first use as a DPP source).
  int s_next = w;
  sfor<0, U>([&](auto uc) {
    issue(uc, s_next);
    s_next += NW;
  });
  {
    constexpr int NQP = (G * E + 15) / 16;
    float qp[NQP * 16];
#pragma unroll
    for (int i = 0; i < NQP * 16; ++i) qp[i] = i < G * E ? qd[i / E][i % E] : 0.f;
#pragma unroll
    for (int c = 0; c < NQP; ++c) pin16<true>(qp + 16 * c);
#pragma unroll
    for (int i = 0; i < G * E; ++i) qd[i / E][i % E] = qp[i];
  }

  auto compute = [&](auto uc) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    const int nr = nrs[u];
    // K elements of row t, dims 64 e + 16 kq + mm (F16 widened, then pinned)
    float kf[E][16];
#pragma unroll
    for (int e = 0; e < E; ++e)
#pragma unroll
      for (int j = 0; j < NK4; ++j) {
        if constexpr (F16) {
          const f16x8 hv = __builtin_bit_cast(f16x8, kb[u][e][j]);
#pragma unroll
          for (int c = 0; c < 8; ++c) kf[e][8 * j + c] = (float)hv[c];
        } else {
          const f32x4 fv = kb[u][e][j];
#pragma unroll
          for (int c = 0; c < 4; ++c) kf[e][4 * j + c] = fv[c];
        }
      }
    if constexpr (F16) {
#pragma unroll
      for (int e = 0; e < E; ++e) pin16<true>(kf[e]);
    }
    // QK partial over this lane's dim block (NPQ partial chains per head),
    // then summed, then across the four blocks.
    float s[G][NPQ];
    sfor<0, 16>([&](auto mc) {
      constexpr int mm = decltype(mc)::value;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int step = mm * E + e;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          if (step < NPQ)
            mul_b<mm>(s[h][step % NPQ], qd[h][e], kf[e][mm]);
          else
            fmac_b<mm>(s[h][step % NPQ], qd[h][e], kf[e][mm]);
        }
      }
    });
    float x[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float a = s[h][0];
#pragma unroll
      for (int pp = 1; pp < NPQ; ++pp) a += s[h][pp];
      x[h] = rows_sum4(a);
    }
    if (nr < kDecodeSub) {
      const bool ok = t < nr;
#pragma unroll
      for (int h = 0; h < G; ++h) x[h] = ok ? x[h] : -INFINITY;
    }
    // A new reference only where a score exceeds the current one.
    float dm = x[0] - m[0];
#pragma unroll
    for (int h = 1; h < G; ++h) dm = fmaxf(dm, x[h] - m[h]);
    if (__builtin_amdgcn_ballot_w64(dm > 0.f) != 0ull) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float mn = fmaxf(m[h], row_max16(x[h]) + kSlack);
        const float al = fast_exp2(m[h] - mn);
        l[h] *= al;
#pragma unroll
        for (int e = 0; e < E; ++e)
#pragma unroll
          for (int pp = 0; pp < NPV; ++pp) O(h, e, pp) *= al;
        m[h] = mn;
      }
    }
    float pb[16];
#pragma unroll
    for (int h = 0; h < 16; ++h) pb[h] = 0.f;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      pb[h] = fast_exp2(x[h] - m[h]);
      l[h] += pb[h];
    }
    // V elements of the 16 rows at this lane's dims
    float vf[E][kDecodeSub];
#pragma unroll
    for (int e = 0; e < E; ++e)
#pragma unroll
      for (int r = 0; r < kDecodeSub; ++r) {
        if constexpr (F16)
          vf[e][r] = (float)__builtin_bit_cast(_Float16, (unsigned short)vb[u][e][r]);
        else
          vf[e][r] = __builtin_bit_cast(float, vb[u][e][r]);
      }
    // every VALU-written operand of the PV multiply-adds (widened V, the
    // probabilities, rescaled accumulators) two wait states behind
    if constexpr (F16) {
#pragma unroll
      for (int e = 0; e < E; ++e) pin16<false>(vf[e]);
    }
#pragma unroll
    for (int c = 0; c < NPIN_O; ++c) pin16<false>(ob + 16 * c);
    pin16<true>(pb);
    sfor<0, 16>([&](auto rc) {
      constexpr int r = decltype(rc)::value;
#pragma unroll
      for (int e = 0; e < E; ++e)
#pragma unroll
        for (int h = 0; h < G; ++h) fmac_b<r>(O(h, e, r % NPV), pb[h], vf[e][r]);
    });
  };

  int s_cur = w;
  const int iters = (mine + U - 1) / U;
  for (int i = 0; i < iters; ++i) {
    sfor<0, U>([&](auto uc) {
      if (s_cur < ns) compute(uc);
      issue(uc, s_next);
      s_cur += NW;
      s_next += NW;
    });
  }

  // The arrival ticket, taken as this wave 0's streaming ends (consumed after
  // the combine).
  unsigned ticket = 0u;
  unsigned* const ctr = cset + (size_t)gid * kCtrInts + kCtrElect;
  if (kpg > 1 && w == 0 && lane == 0)
    ticket = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // This wave's partial into LDS: l summed over the row's positions (rows
  // are replicas), o as it lies.
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float ls = row_sum16s(l[h]);
    if (lane == 0) {
      wm[w][h] = m[h];
      wl[w][h] = ls;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float a = O(h, e, 0);
#pragma unroll
      for (int pp = 1; pp < NPV; ++pp) a += O(h, e, pp);
      wo[w][h][64 * e + 16 * kq + t] = a;
    }
  }
  __syncthreads();

  // The workgroup's partial for output (h, d) = (i / D, i % D), waves merged
  // in wave order.
  constexpr int NI = (G * D + NT - 1) / NT;
  float num[NI], mx[NI], den[NI];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const int i = threadIdx.x + k * NT;
    num[k] = 0.f;
    den[k] = 0.f;
    mx[k] = -INFINITY;
    if (i < G * D) {
      const int h = i / D, d = i - h * D;
      float M = -INFINITY;
#pragma unroll
      for (int v = 0; v < NW; ++v) M = fmaxf(M, wm[v][h]);
      float a = 0.f, b = 0.f;
#pragma unroll
      for (int v = 0; v < NW; ++v) {
        const float f = fast_exp2(wm[v][h] - M);  // 0 for a wave with no positions
        a += f * wo[v][h][d];
        b += f * wl[v][h];
      }
      num[k] = a;
      den[k] = b;
      mx[k] = M;
    }
  }
  auto write_out = [&](int i, float a, float b) __attribute__((always_inline)) {
    const int h = i / D, d = i - h * D;
    if (h < Gc)
      gstore<float>(reinterpret_cast<char*>(it.out) + (int64_t)(head0 + h) * it.o_s1 + 4 * d, a / b);
  };
  if (kpg == 1) {
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      const int i = threadIdx.x + k * NT;
      if (i < G * D) write_out(i, num[k], den[k]);
    }
    return;
  }

  // Record words: [i < G D] numerators, then m[h], then the sums l[h].
  constexpr int RW = G * D + 2 * G;
  const uint64_t stamp = (uint64_t)epoch << 32;
  uint64_t* const rec = reinterpret_cast<uint64_t*>(p.rec);
  const size_t slot_words = p.rec_words;
  {
    uint64_t* const mine_rec = rec + (size_t)wg * slot_words;
#pragma unroll
    for (int k = 0; k < NI; ++k) {
      const int i = threadIdx.x + k * NT;
      if (i < G * D) {
        __hip_atomic_store(mine_rec + i, stamp | __float_as_uint(num[k]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int h = i / D;
        if (i - h * D == 0) {
          __hip_atomic_store(mine_rec + G * D + h, stamp | __float_as_uint(mx[k]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(mine_rec + G * D + G + h, stamp | __float_as_uint(den[k]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
  if (w == 0 && lane == 0) merge_flag = ticket == (unsigned)(kpg - 1) ? 1u : 0u;
  __syncthreads();
  if (!merge_flag) return;

  // The merge: every part's record in part order (this part's own values in
  // its place), each word polled until it carries this launch's stamp.
  uint64_t* const grec = rec + (size_t)(it.wg0 + gl * kpg) * slot_words;
  const int max_polls = p.max_polls;
  bool lost = false;
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const int i = threadIdx.x + k * NT;
    if (i >= G * D) continue;
    const int h = i / D;
    float Mc = -INFINITY, a = 0.f, b = 0.f;
    constexpr int CH = 8;  // parts whose words are requested together
    for (int q0 = 0; q0 < kpg; q0 += CH) {
      uint64_t wn[CH], wmx[CH], wd[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int q = q0 + c;
        if (q < kpg && q != part) {
          const uint64_t* r = grec + (size_t)q * slot_words;
          wn[c] = __hip_atomic_load(r + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          wmx[c] = __hip_atomic_load(r + G * D + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          wd[c] = __hip_atomic_load(r + G * D + G + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          wn[c] = wmx[c] = wd[c] = stamp;
        }
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int q = q0 + c;
        if (q >= kpg) continue;
        float vn, vm, vd;
        if (q == part) {
          vn = num[k];
          vm = mx[k];
          vd = den[k];
        } else {
          const uint64_t* r = grec + (size_t)q * slot_words;
          int n = 0;
          while (((unsigned)(wn[c] >> 32) != epoch || (unsigned)(wmx[c] >> 32) != epoch ||
                  (unsigned)(wd[c] >> 32) != epoch) &&
                 n < max_polls) {
            __builtin_amdgcn_s_sleep(1);
            wn[c] = __hip_atomic_load(r + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wmx[c] = __hip_atomic_load(r + G * D + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wd[c] = __hip_atomic_load(r + G * D + G + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ++n;
          }
          if ((unsigned)(wn[c] >> 32) != epoch || (unsigned)(wmx[c] >> 32) != epoch ||
              (unsigned)(wd[c] >> 32) != epoch)
            lost = true;
          vn = __uint_as_float((unsigned)wn[c]);
          vm = __uint_as_float((unsigned)wmx[c]);
          vd = __uint_as_float((unsigned)wd[c]);
        }
        const float Mn = fmaxf(Mc, vm);
        const float fa = fast_exp2(Mc - Mn), fb = fast_exp2(vm - Mn);
        a = a * fa + vn * fb;
        b = b * fa + vd * fb;
        Mc = Mn;
      }
    }
    write_out(i, lost ? NAN : a, lost ? 1.f : b);
  }
  if (lost) __hip_atomic_fetch_add(p.status + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  (void)RW;
}

namespace {

template <int E, typename KT, int G>
hipError_t launch_stream_g(const DecodeParams& p, int grid_x, int n_items, hipStream_t stream) {
  constexpr int NW = 8;
  constexpr int U = 2;
  hipLaunchKernelGGL((stream_decode_kernel<E, KT, G, NW, U>), dim3((unsigned)grid_x, (unsigned)n_items),
                     dim3(NW * kWave), 0, stream, p);
  return hipGetLastError();
}

template <int E, typename KT>
hipError_t launch_stream_e(const DecodeParams& p, int grid_x, int n_items, int group, hipStream_t stream) {
  switch (group) {
    case 1: return launch_stream_g<E, KT, 1>(p, grid_x, n_items, stream);
    case 2: return launch_stream_g<E, KT, 2>(p, grid_x, n_items, stream);
    case 3: return launch_stream_g<E, KT, 3>(p, grid_x, n_items, stream);
    case 4: return launch_stream_g<E, KT, 4>(p, grid_x, n_items, stream);
    case 5: return launch_stream_g<E, KT, 5>(p, grid_x, n_items, stream);
    case 6: return launch_stream_g<E, KT, 6>(p, grid_x, n_items, stream);
    case 7: return launch_stream_g<E, KT, 7>(p, grid_x, n_items, stream);
    case 8: return launch_stream_g<E, KT, 8>(p, grid_x, n_items, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

size_t stream_record_words(int head_dim, int group) { return (size_t)group * head_dim + 2 * (size_t)group; }

hipError_t launch_stream_decode(const DecodeParams& p, int grid_x, int n_items, int head_dim, bool f16, int group,
                                hipStream_t stream) {
  if (grid_x < 1 || n_items < 1 || n_items > kDecodeMaxItems) return hipErrorInvalidValue;
  if (head_dim == 64)
    return f16 ? launch_stream_e<1, _Float16>(p, grid_x, n_items, group, stream)
               : launch_stream_e<1, float>(p, grid_x, n_items, group, stream);
  if (head_dim == 128)
    return f16 ? launch_stream_e<2, _Float16>(p, grid_x, n_items, group, stream)
               : launch_stream_e<2, float>(p, grid_x, n_items, group, stream);
  return hipErrorInvalidValue;
}

}  // namespace mi
