// mul_mat.hip -- the step after attention on the device: MI_OP_QUANTIZE_Q8_0
// (src/ops_cpu.cpp:462-479 -> src/quant.cpp:188-210) and MI_OP_MUL_MAT with
// Q8_0 weights (src/ops_cpu.cpp:226-236), e.g. the attention output
// projection. HBM-bound matrix-vector work: the weights are read once per
// launch; a decode column reuses nothing else.
//
// Both reproduce the engine bit for bit:
//  - activation blocks of 32: amax by a strict greater-than scan, d = amax /
//    127 and id = 1 / d as correctly rounded float divisions, q = rint(x id)
//    (round half to even, as lrintf) clamped to [-127, 127];
//  - the dot product of a weight row and an activation column in the order
//    of the reference's default (AVX2 + FMA) path: accumulator l (0..7) takes
//    fma(float(int8 dot of bytes 4l..4l+3 of each block), fp16(w.d) * a.d,
//    acc_l) block by block (v_dot4 gives that byte group's exact int32 sum),
//    then ((acc0 + acc4) + (acc1 + acc5)) + ((acc2 + acc6) + (acc3 + acc7)).
//    Lane l of an 8-lane group owns accumulator l; the horizontal sum is two
//    xor exchanges (float addition is commutative, so each partial is the
//    same value on both lanes that form it).
#include <algorithm>
#include <type_traits>

#include "attn_common.h"
#include "kernels.h"

#define MI_LIBM_HD __host__ __device__
#include "libm_ref.h"

namespace mi {
namespace {
__constant__ uint64_t kExpfTab[32] = MI_EXPF_TABLE;
}  // namespace

// SiLU(g) * u as the engine computes it: g / (1 + expf(-g)) with the host C
// library's expf (libm_ref.h, its table at tab), then the product.
template <typename Tab>
__device__ inline float swiglu_value(float g, float u, Tab tab) {
#pragma clang fp contract(off)
  return (g / (1.0f + expf_ref(-g, tab))) * u;
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// The horizontal sum of an 8-lane row group's accumulators in the order of the
// reference's AVX2 reduction, ((a0 + a4) + (a1 + a5)) + ((a2 + a6) + (a3 + a7)),
// on every lane of the group (float addition is commutative, so both lanes of
// a pair form the same value). The partners come by DPP moves, not the LDS
// pipe: lane l ^ 4 by a row shift (left for l & 4 == 0, right otherwise), then
// quad swaps for l ^ 1 and l ^ 2.
__device__ inline float q8_hsum8(float a, int lane) {
#pragma clang fp contract(off)
  const float up = dpp_mov<0x104>(a), down = dpp_mov<0x114>(a);  // row_shl:4, row_shr:4
  float t = a + ((lane & 4) ? down : up);
  t = t + dpp_mov<0xB1>(t);  // quad_perm [1,0,3,2]
  return t + dpp_mov<0x4E>(t);  // quad_perm [2,3,0,1]
}
// Row group rs ^ 1's value (8 lanes away): a row rotation by 8.
__device__ inline float q8_xor8(float a) { return dpp_mov<0x128>(a); }

// One thread per 32-element block of one activation row.
__global__ void quantize_q8_0_act_kernel(const Q8Quantize p) {
#pragma clang fp contract(off)
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nb = p.ne0 / 32;
  if (idx >= p.rows * nb) return;
  const int64_t r = idx / nb, b = idx - r * nb;
  const int64_t i1 = r % p.ne1, i2 = (r / p.ne1) % p.ne2, i3 = r / (p.ne1 * p.ne2);
  const float* x = reinterpret_cast<const float*>(p.src + i1 * p.src_nb[1] + i2 * p.src_nb[2] +
                                                  i3 * p.src_nb[3]) + 32 * b;
  float v[32];
#pragma unroll
  for (int j = 0; j < 32; ++j) v[j] = gload<float>(x + j);  // rows are 4-byte aligned only
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const float av = fabsf(v[j]);
    if (av > amax) amax = av;
  }
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  char* y = p.dst + i1 * p.dst_nb[1] + i2 * p.dst_nb[2] + i3 * p.dst_nb[3] + 36 * b;
  gstore<float>(y, d);
#pragma unroll
  for (int j = 0; j < 32; j += 4) {
    unsigned word = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      int q = (int)__builtin_rintf(v[j + t] * id);
      q = q > 127 ? 127 : (q < -127 ? -127 : q);
      word |= (unsigned)(q & 0xff) << (8 * t);
    }
    gstore<unsigned>(y + 4 + j, word);
  }
}

// Rows of 8 lanes (32 rows per 256-thread workgroup); columns in chunks of
// kQ8Cols, each lane keeping its accumulator for every column of the chunk.
constexpr int kQ8Cols = 8;

__global__ __launch_bounds__(256) void mul_mat_q8_0_kernel(const Q8MulMat p) {
#pragma clang fp contract(off)
  const int l = threadIdx.x & 7;
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const bool live = row < p.n;  // dead lanes still join the exchanges
  const char* w = p.w + (live ? row : 0) * p.w_nb1;
  const int nblk = (int)(p.k / 32);
  for (int64_t c0 = 0; c0 < p.m; c0 += kQ8Cols) {
    const int nc = (int)min<int64_t>(kQ8Cols, p.m - c0);
    float acc[kQ8Cols];
#pragma unroll
    for (int c = 0; c < kQ8Cols; ++c) acc[c] = 0.0f;
    for (int b = 0; b < nblk; ++b) {
      const char* wb = w + 34 * (int64_t)b;
      // 34-byte blocks: the scale and the byte group are 2-byte aligned
      const float wd = (float)__builtin_bit_cast(_Float16, gload<unsigned short>(wb));
      const int wq = (int)((unsigned)gload<unsigned short>(wb + 2 + 4 * l) |
                           ((unsigned)gload<unsigned short>(wb + 4 + 4 * l) << 16));
#pragma unroll
      for (int c = 0; c < kQ8Cols; ++c) {
        if (c < nc) {
          const char* ab = p.a + (c0 + c) * p.a_nb1 + 36 * (int64_t)b;
          const float dxdy = wd * gload<float>(ab);
          const int isum = __builtin_amdgcn_sdot4(wq, gload<int>(ab + 4 + 4 * l), 0, false);
          acc[c] = __builtin_fmaf((float)isum, dxdy, acc[c]);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < kQ8Cols; ++c) {
      if (c < nc) {
        // lanes l and l^4 -> acc_l + acc_(l+4); then pairs; lane 0 holds
        // ((acc0 + acc4) + (acc1 + acc5)) + ((acc2 + acc6) + (acc3 + acc7))
        float s = q8_hsum8(acc[c], threadIdx.x);
        if (live && l == 0) {
          if (p.add) s = s + gload<float>(p.add + row * p.add_nb0 + (c0 + c) * p.add_nb1);
          gstore<float>(p.dst + q8_unperm_row(row, p.perm_hd, p.perm_rows) * p.dst_nb0 + (c0 + c) * p.dst_nb1, s);
        }
      }
    }
  }
}

// The streaming form, for weight rows of at most 1 KB (k <= 960: every matrix
// of a 896-wide model), 16-byte aligned groups of 8 rows and M <= kQ8Cols
// columns. One workgroup of 8 waves per CU; each wave walks row groups (8
// rows) g = wave_id, wave_id + stride, ... through a ring of 2 LDS slots
// filled by buffer_load ... lds (16 bytes per lane, one resource per group
// bounded at the tensor's end, so bytes past it arrive as zeros without a
// request, and a group past the end refills through a zero-sized resource).
// Its 8-lane row groups read their byte groups back from the slot. Per
// iteration a wave issues exactly M stores then 8 loads, so the wait for a
// slot is the fixed vmcnt(M + 8) (vmcnt(8) the first time).
constexpr int kQ8RowBytesMax = 1024;
constexpr int kQ8RingWaves = 8;
constexpr int kQ8Slot = 8 * kQ8RowBytesMax;
constexpr int kQ8MaxBlocks = 30;                   // k <= 960
constexpr int kQ8ActBytesMax = kQ8Cols * kQ8MaxBlocks * 36;
constexpr int kQ8RingTake = kQ8RingWaves * 2 * kQ8Slot + kQ8ActBytesMax;  // the group counter
constexpr int kQ8Scale = kQ8RingTake + 16;        // the norm scale of each column
constexpr int kQ8RingLds = kQ8Scale + 4 * kQ8Cols;
constexpr int kQ8XOff = kQ8RingLds;                // one F32 column's squares (M = 1), past the ring,
constexpr int kQ8SqN = 8 * 128;                    // padded to the 8 waves' segments of 128
constexpr int kQ8SumWork = kQ8XOff + 4 * kQ8SqN;   // the 8-wave ordered sum's work area
constexpr int kQ8SwTab = kQ8SumWork + 64 + 8 * kWave * 4;  // SwiGLU epilogue: expf's table
constexpr int kQ8SwVals = kQ8SwTab + 32 * 8;                 // and the workgroup's 32 values
constexpr int kQ8RingLdsAll = kQ8SwVals + 32 * 4;

// A load of two floats that the compiler does not track, so that it never
// makes the products wait for it (its register allocation otherwise sometimes
// reuses a register of the pending load at once); landed(v) waits for every
// load of the wave (vmcnt 0) and ties v to that wait, so nothing reads v
// earlier. Issue it on every path: a branch around it could make the compiler
// copy the register before the data has landed.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ inline f32x2_t load_f32x2_async(const float* p) {
  f32x2_t v;
  asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ inline void landed(f32x2_t& v) { asm volatile("s_waitcnt vmcnt(0)" : "+v"(v)::"memory"); }
// vmcnt(BASE + extra) for extra in [0, 3] (a uniform value)
template <int BASE>
__device__ inline void wait_vmem_plus(int extra) {
  if (extra == 0)
    wait_vmem<BASE>();
  else if (extra == 1)
    wait_vmem<BASE + 1>();
  else if (extra == 2)
    wait_vmem<BASE + 2>();
  else
    wait_vmem<BASE + 3>();
}

// Returns *c and adds 1 (an LDS atomic). As asm: the compiler's wait insertion
// would otherwise wait for every LDS-direct load in flight (vmcnt(0)) before
// an LDS atomic. The counter is never a load target.
__device__ inline unsigned lds_take(__attribute__((address_space(3))) unsigned* c) {
  unsigned t;
  asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)" : "=v"(t) : "v"(c), "v"(1u) : "memory");
  return t;
}

// EPI: the stacked Q/K/V epilogue (rows permuted within heads; RoPE and the
// K/V append for one column) -- a separate instantiation, so the plain form
// carries none of it.
template <int M, bool EPI>
__global__ __launch_bounds__(kQ8RingWaves * kWave) void mul_mat_q8_0_ring_kernel(const Q8MulMat p) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) char ring_lds[];
  lds_t* const lds = (lds_t*)ring_lds;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nblk = (int)(p.k / 32);
  const int abytes = nblk * 36;
  char* const act_lds = ring_lds + kQ8RingWaves * 2 * kQ8Slot;
  // This workgroup's contiguous range of 8-row groups; its waves take groups
  // from an LDS counter as they refill, so a wave served faster takes more
  // and the waves finish together.
  const int64_t n_groups = (p.n + 7) / 8;
  const int64_t glo = n_groups * blockIdx.x / gridDim.x;
  const int64_t ngw = n_groups * (blockIdx.x + 1) / gridDim.x - glo;
  __attribute__((address_space(3))) unsigned* const take =
      reinterpret_cast<__attribute__((address_space(3))) unsigned*>(lds + kQ8RingTake);
  const int64_t total = p.n * p.w_nb1;
  const rsrc_t none = make_rsrc(p.w, 0u);
  lds_t* const slots = lds + wv * 2 * kQ8Slot;
  // refills slot s with the next group taken; returns it, or -1 past the
  // range (with issue_dead, a take past the range still issues its 8
  // zero-sized requests, keeping the number of loads per refill fixed)
  auto refill = [&](int s, bool issue_dead) __attribute__((always_inline)) -> int64_t {
    unsigned t = 0;
    if (lane == 0) t = lds_take(take);
    t = (unsigned)__builtin_amdgcn_readfirstlane((int)t);
    const int64_t g = glo + (int64_t)t;
    const bool live = t < (unsigned)ngw;
    rsrc_t r = none;
    if (live) {
      const int64_t start = g * 8 * p.w_nb1;
      r = make_rsrc(p.w + start, (unsigned)min<int64_t>(8 * p.w_nb1, total - start));
    }
    if (live || issue_dead) {
#pragma unroll
      for (int i = 0; i < 8; ++i) dma16(r, slots + s * kQ8Slot + 1024 * i, (unsigned)(1024 * i + 16 * lane));
    }
    return live ? g : -1;
  };
  int64_t g_0, g_1;  // the group in each slot, or -1
  // LDS read through lds_t pointers into the regions past the ring: the
  // compiler then sees that they cannot overlap the ring's LDS-direct
  // requests and does not wait for those before reading
  lds_t* const s_scale = lds + kQ8Scale;
  if constexpr (M == 1) {
    // One column: its loads go into registers (at most 2 elements, or 1
    // activation word, per thread: k <= 960), the ring's first requests
    // follow, and the prologue's arithmetic runs under their latency. The
    // column's squares are staged past the ring for the norm's ordered sum.
    constexpr int kT = kQ8RingWaves * kWave;
    const int t = threadIdx.x;
    const int k = (int)p.k;
    float xv[2] = {0.0f, 0.0f}, nw[2] = {1.0f, 1.0f};
    unsigned av = 0;
    // the SwiGLU epilogue reads expf's table from LDS (a read of the
    // __constant__ one is a global load, whose wait would drain the ring)
    const uint64_t te = p.swiglu_out ? kExpfTab[lane & 31] : 0;
    if (p.x) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (t + kT * j < k) {
          xv[j] = gload<float>(p.x + t + kT * j);
          if (p.norm_w) nw[j] = gload<float>(p.norm_w + t + kT * j);
        }
    } else if (t < abytes / 4) {
      av = gload<unsigned>(p.a + 4 * t);
    }
    if (t == 0) *take = 0u;
    // the region's blocks past the row are zero: their products add exactly
    // +0.0 (the weight block read for them is a real one, so its scale is
    // finite, and a sum is never -0.0), so no block needs a select
    for (int i = t; i < (kQ8MaxBlocks - nblk) * 9; i += kT)
      *reinterpret_cast<unsigned*>(act_lds + abytes + 4 * i) = 0u;
    wg_barrier();  // the counter is zero (the loads above stay in flight)
    // slot 0 is requested even for an empty take, so that exactly 8
    // requests follow the loads above: the compiler's wait for them (at the
    // empty asm, which reads them all) is vmcnt(8). Then slot 1, with no
    // requests for an empty take (a wave with one group has nothing to issue
    // there): its count is known only at run time, and the loads above are
    // no longer waited for after it.
    g_0 = refill(0, true);
    asm volatile("" ::"v"(xv[0]), "v"(xv[1]), "v"(nw[0]), "v"(nw[1]), "v"(av), "v"(te));
    g_1 = refill(1, false);
    if (!p.x) {
      if (t < abytes / 4) *reinterpret_cast<unsigned*>(act_lds + 4 * t) = av;
    } else {
      float scale = 1.0f;
      if (p.norm_w) {
        // the squares, padded with +0.0 to kQ8SqN; their sum in the
        // reference's order, formed by the 8 waves together
        static_assert(kQ8RingWaves == 8 && 2 * kT == kQ8SqN, "8 waves, two squares per thread");
        lds_t* const sq = lds + kQ8XOff;
#pragma unroll
        for (int j = 0; j < 2; ++j) lds_store<float>(sq + 4 * (t + kT * j), t + kT * j < k ? xv[j] * xv[j] : 0.0f);
        wg_barrier();
        scale = rms_scale(ordered_sum_lds_8waves<kQ8SqN / 8>(sq, lds + kQ8SumWork, wv, lane), k, p.eps);
      }
      // one thread per element in groups of 32 lanes forming each block (k
      // and kT are multiples of 32, so a group is active as a whole)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int e = t + kT * j;
        if (e < k) {
          const float y = p.norm_w ? (xv[j] * scale) * nw[j] : xv[j];
          float d;
          const int q = q8_lane_quant(y, d);
          char* blk = act_lds + 36 * (e / 32);
          if ((e & 31) == 0) *reinterpret_cast<float*>(blk) = d;
          blk[4 + (e & 31)] = (char)q;
        }
      }
    }
    if (p.swiglu_out && t < 32) lds_store<uint64_t>(lds + kQ8SwTab + 8 * t, te);
    wg_barrier();  // the activation (and expf's table) is staged
  } else {
    if (!p.x) {
      for (int i = threadIdx.x; i < M * abytes / 4; i += kQ8RingWaves * kWave) {
        const int c = i / (abytes / 4), o = 4 * (i - c * (abytes / 4));
        *reinterpret_cast<unsigned*>(act_lds + c * abytes + o) = gload<unsigned>(p.a + c * p.a_nb1 + o);
      }
    } else {
      // the prologue: columns into LDS (the ring slots are free until the
      // first refill), the norm's ordered sums, then one thread per element
      // in groups of 32 lanes forming each block
      float* const xs = reinterpret_cast<float*>(ring_lds);
      float* const sq = xs + M * p.k;
      const int k = (int)p.k;
      for (int i = threadIdx.x; i < M * k; i += kQ8RingWaves * kWave) {
        const int c = i / k;
        const float v = gload<float>(p.x + c * p.x_ld + (i - c * k));
        xs[i] = v;
        sq[i] = v * v;
      }
      __syncthreads();
      if (p.norm_w && threadIdx.x < M)
        lds_store<float>(s_scale + 4 * threadIdx.x, rms_scale(ordered_sum(sq + threadIdx.x * k, k), k, p.eps));
      __syncthreads();
      for (int i = threadIdx.x; i < M * k; i += kQ8RingWaves * kWave) {
        const int c = i / k, e = i - c * k;
        const float y = p.norm_w ? (xs[i] * lds_load<float>(s_scale + 4 * c)) * gload<float>(p.norm_w + e) : xs[i];
        float d;
        const int q = q8_lane_quant(y, d);
        char* blk = act_lds + c * abytes + 36 * (e / 32);
        if ((e & 31) == 0) *reinterpret_cast<float*>(blk) = d;
        blk[4 + (e & 31)] = (char)q;
      }
    }
    if (threadIdx.x == 0) *take = 0u;
    __syncthreads();  // the activation is staged (before the ring requests: the barrier waits for all loads)
    g_0 = refill(0, true);
    g_1 = refill(1, true);
  }
  const int l = lane & 7, rs = lane >> 3;
  const lds_t* const act = lds + kQ8RingWaves * 2 * kQ8Slot;
  // one column: this lane's activation byte groups and the block scales, in registers
  float a_d[M == 1 ? kQ8MaxBlocks : 1];
  int a_q[M == 1 ? kQ8MaxBlocks : 1];
  if constexpr (M == 1) {
    // every block of the region, read without branches so that the reads
    // are all in flight together (the blocks past the row are zero)
#pragma unroll
    for (int b = 0; b < kQ8MaxBlocks; ++b) {
      a_d[b] = lds_load<float>(act + 36 * b);
      a_q[b] = lds_load<int>(act + 36 * b + 4 + 4 * l);
    }
  }
  // slots in turn until the first empty one (a wave's takes increase, so
  // every later slot is empty too)
  const bool one_slot = M == 1 && g_1 < 0;  // the first fill issued slot 0's requests only
  for (int s = 0, it = 0;; s ^= 1, ++it) {
    const int64_t g = s ? g_1 : g_0;
    if (g < 0) break;
    const lds_t* const w = lds + (wv * 2 + s) * kQ8Slot + rs * (int)p.w_nb1;
    const int64_t row = g * 8 + rs;
    // the optional added term (and, for the RoPE epilogue, the row's cos/sin
    // pair): with one column requested before the slot's wait, so that their
    // latency overlaps it and the products; counted in that wait (extra).
    // Every lane loads, from a row inside the tensor. The pair is an asm load
    // issued on every path (no branch, so the compiler never copies its
    // register before landed() waits for it); its wait drains the wave.
    float addv[M];
    f32x2_t csv;
    int extra = 0;
    if constexpr (M == 1) {
      if (p.add) {
        addv[0] = gload<float>(p.add + min(row, p.n - 1) * p.add_nb0);
        ++extra;
      }
      if constexpr (EPI) {
        const RopeEpi& re = p.rope;
        const int64_t pair = p.rope_on ? (int64_t)re.pos * (re.hd / 2) + (row % re.hd) / 2 : 0;
        csv = load_f32x2_async(p.rope_on ? re.cs + 2 * pair : reinterpret_cast<const float*>(p.w));
        ++extra;
      }
    }
    // (the SwiGLU epilogue issues no stores: it writes LDS)
    if (it == 0 && one_slot)
      wait_vmem_plus<0>(extra);
    else if (it == 0)
      wait_vmem_plus<8>(extra);
    else if (M == 1 && p.swiglu_out)
      wait_vmem_plus<8>(extra);
    else
      wait_vmem_plus<M + 8>(extra);
    if constexpr (M > 1) {
      // more columns: requested after the wait, their latency overlapping
      // the products
      if (p.add) {
        const int64_t ra = min(row, p.n - 1);
#pragma unroll
        for (int c = 0; c < M; ++c) addv[c] = gload<float>(p.add + ra * p.add_nb0 + c * p.add_nb1);
      }
    }
    float acc[M];
#pragma unroll
    for (int c = 0; c < M; ++c) acc[c] = 0.0f;
    // blocks fully unrolled (k <= 960), used in order; the LDS reads of all
    // of them can be issued ahead of the chain of multiply-adds
#pragma unroll
    for (int b = 0; b < kQ8MaxBlocks; ++b) {
      const int bb = min(b, nblk - 1);  // reads stay in the row; blocks past it are not added
      const lds_t* wb = w + 34 * bb;
      const float wd = (float)__builtin_bit_cast(_Float16, lds_load<unsigned short>(wb));
      const int wq = (int)((unsigned)lds_load<unsigned short>(wb + 2 + 4 * l) |
                           ((unsigned)lds_load<unsigned short>(wb + 4 + 4 * l) << 16));
#pragma unroll
      for (int c = 0; c < M; ++c) {
        const float dxdy = wd * (M == 1 ? a_d[b] : lds_load<float>(act + c * abytes + 36 * bb));
        const int aq = M == 1 ? a_q[b] : lds_load<int>(act + c * abytes + 36 * bb + 4 + 4 * l);
        const int isum = __builtin_amdgcn_sdot4(wq, aq, 0, false);
        const float r = __builtin_fmaf((float)isum, dxdy, acc[c]);
        acc[c] = M == 1 || b < nblk ? r : acc[c];
      }
    }
#pragma unroll
    for (int c = 0; c < M; ++c) {
      const float t = q8_hsum8(acc[c], lane);
      acc[c] = t;
    }
    // the added term's loads finish (vmcnt 0, which also drains the other
    // slot's refill) before the stores, so the fixed waits still count
    // exactly M stores and 8 loads per iteration
    if (p.add) {
      wait_vmem<0>();
#pragma unroll
      for (int c = 0; c < M; ++c)
        if (row < p.n && l == 0) acc[c] = acc[c] + addv[c];
    }
    if constexpr (EPI && M == 1) landed(csv);
    // RoPE epilogue (one column): the rotation partner is row rs ^ 1 of this
    // group, 8 lanes away; the destination is chosen per lane, so it is still
    // one store instruction
    float* dst_rope = nullptr;
    if constexpr (EPI && M == 1) {
      if (p.rope_on) {
        const RopeEpi& re = p.rope;
        const float other = q8_xor8(acc[0]);
        const int64_t qk_rows = (int64_t)re.n_q + re.n_kv;
        const int64_t h = row / re.hd;  // head (Q heads, then K heads, then V heads)
        const int w = (int)(row - h * re.hd);
        if (row < qk_rows) {
          const float x0 = (w & 1) ? other : acc[0], x1 = (w & 1) ? acc[0] : other;
          acc[0] = (w & 1) ? x0 * csv.y + x1 * csv.x : x0 * csv.x - x1 * csv.y;
        }
        const int d = row < qk_rows ? (w >> 1) + (w & 1) * (re.hd / 2) : w;
        if (row < re.n_q)
          dst_rope = re.q_out + h * re.hd + d;
        else if (row < qk_rows)
          dst_rope = reinterpret_cast<float*>(re.k_row + (h - re.n_q / re.hd) * re.c_s1) + d;
        else
          dst_rope = reinterpret_cast<float*>(re.v_row + (h - qk_rows / re.hd) * re.c_s1) + d;
      }
    }
    // the slot's reads are done before it is refilled; then M stores (row 0
    // of a group always exists, so every store instruction issues), 8 loads
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (M == 1 && p.swiglu_out) {
      // gate rows are even, their up rows 8 lanes away: the group's 4 values
      // go to the workgroup's block in LDS (the workgroup's groups are the
      // block's 8)
      const float up = q8_xor8(acc[0]);
      if ((rs & 1) == 0 && l == 0)
        lds_store<float>(lds + kQ8SwVals + 4 * (4 * (int)(g - glo) + (rs >> 1)),
                         swiglu_value(acc[0], up, (const __attribute__((address_space(3))) uint64_t*)(lds + kQ8SwTab)));
    } else {
#pragma unroll
    for (int c = 0; c < M; ++c) {
      float* const o = !EPI ? reinterpret_cast<float*>(p.dst + row * p.dst_nb0 + c * p.dst_nb1)
                       : dst_rope ? dst_rope
                                  : reinterpret_cast<float*>(p.dst + q8_unperm_row(row, p.perm_hd, p.perm_rows) * p.dst_nb0 + c * p.dst_nb1);
      if (row < p.n && l == 0) gstore<float>(o, acc[c]);
    }
    }
    const int64_t gn = refill(s, true);
    if (s)
      g_1 = gn;
    else
      g_0 = gn;
  }
  wait_vmem<0>();
  if (M == 1 && p.swiglu_out) {
    // the block: its 32 values in element order, quantised by 32 lanes
    wg_barrier();
    if (wv == 0 && lane < 32) {
      float d;
      const int q = q8_lane_quant(lds_load<float>(lds + kQ8SwVals + 4 * lane), d);
      char* const blk = p.swiglu_out + 36 * (int64_t)blockIdx.x;
      if (lane == 0) gstore<float>(blk, d);
      gstore<signed char>(blk + 4 + lane, (signed char)q);
    }
  }
}

// The staged form, for rows longer than the ring's slots (e.g. a 4864-wide
// FFN down projection) and for more than kQ8Cols columns (a prompt's
// tokens): one wave per group of 8 rows copies the group's rows (contiguous
// in memory) into LDS with 16-byte loads, then, per chunk of up to kQ8Cols
// columns, stages the chunk's activation blocks beside them; lane (row r =
// lane / 8, accumulator l = lane % 8) walks its row's blocks in order from
// LDS. Weights are read from HBM once however many columns there are.
constexpr int kQ8StageLdsMax = 96 * 1024;

__host__ __device__ inline int64_t round1k(int64_t n) { return (n + 1023) & ~int64_t(1023); }
// LDS of the staged form: the 8-row group and one chunk of activation columns,
// each rounded up to whole 1 KB LDS-direct transfers.
__host__ __device__ inline int64_t q8_stage_lds_bytes(int64_t w_nb1, int64_t k) {
  return round1k(8 * w_nb1) + round1k(kQ8Cols * (k / 32) * 36);
}

// MC: columns per chunk (the host picks min(m, kQ8Cols)); only the last chunk
// may be partial.
template <int MC>
__global__ __launch_bounds__(kWave) void mul_mat_q8_0_staged_kernel(const Q8MulMat p) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) char stage_lds[];
  const lds_t* const lds = (const lds_t*)stage_lds;
  const int lane = threadIdx.x;
  const int64_t g = blockIdx.x;
  const int nrows = (int)min<int64_t>(8, p.n - g * 8);
  // the group's bytes end at its last row's last block (rows may be padded)
  const int64_t wbytes = (nrows - 1) * p.w_nb1 + p.k / 32 * 34;  // a multiple of 2
  const char* const wsrc = p.w + g * 8 * p.w_nb1;
  // the group's rows straight into LDS, every 1 KB transfer in flight at once
  // (bytes past the group arrive as zeros from the bounded resource). The
  // resource's range check is per dword, so it ends at the last whole dword;
  // a 2-byte tail is copied separately once the transfers have landed.
  const int64_t wb4 = wbytes & ~int64_t(3);
  {
    const rsrc_t r = make_rsrc(wsrc, (unsigned)wb4);
    const int n1k = (int)((wbytes + 1023) / 1024);
    for (int i = 0; i < n1k; ++i) dma16(r, (lds_t*)stage_lds + 1024 * i, (unsigned)(1024 * i + 16 * lane));
  }
  const int nblk = (int)(p.k / 32);
  const int abytes = nblk * 36;
  const int64_t act_off = round1k(8 * p.w_nb1);
  // contiguous 16-byte aligned columns: a chunk is one range, loaded the same way
  const bool act_dma = p.a_nb1 == abytes && abytes % 16 == 0 && reinterpret_cast<uintptr_t>(p.a) % 16 == 0;
  const int l = lane & 7, r = lane >> 3;
  const int64_t row = g * 8 + r;
  const bool live = r < nrows;
  const lds_t* const w = lds + (live ? r : 0) * p.w_nb1;
  for (int64_t c0 = 0; c0 < p.m; c0 += MC) {
    const int nc = (int)min<int64_t>(MC, p.m - c0);
    __syncthreads();  // the previous chunk's activation reads are done
    if (act_dma) {
      const int64_t bytes = (int64_t)nc * abytes;
      const rsrc_t r = make_rsrc(p.a + c0 * p.a_nb1, (unsigned)bytes);
      const int n1k = (int)((bytes + 1023) / 1024);
      for (int i = 0; i < n1k; ++i)
        dma16(r, (lds_t*)stage_lds + act_off + 1024 * i, (unsigned)(1024 * i + 16 * lane));
    } else {
      for (int i = lane; i < nc * abytes / 4; i += kWave) {
        const int c = i / (abytes / 4), o = 4 * (i - c * (abytes / 4));
        lds_store<unsigned>((lds_t*)(stage_lds + act_off + c * abytes + o),
                            gload<unsigned>(p.a + (c0 + c) * p.a_nb1 + o));
      }
    }
    // one column: the added term is requested now, so its latency overlaps
    // the transfers'
    float addv = 0.0f;
    if (MC == 1 && p.add) addv = gload<float>(p.add + min(row, p.n - 1) * p.add_nb0 + c0 * p.add_nb1);
    wait_vmem<0>();  // the LDS-direct transfers (and the added term) have landed
    if (c0 == 0 && wb4 != wbytes && lane == 0)
      lds_store<unsigned short>((lds_t*)(stage_lds + wb4), gload<unsigned short>(wsrc + wb4));
    __syncthreads();
    float acc[MC];
#pragma unroll
    for (int c = 0; c < MC; ++c) acc[c] = 0.0f;
    const lds_t* const act = lds + act_off + 4 + 4 * l;
    // blocks in order; 8 at a time with all their LDS reads issued first, so
    // their latency overlaps the chain of multiply-adds (a tail of fewer than
    // 8 re-reads the last block and does not add it)
    for (int b0 = 0; b0 < nblk; b0 += 8) {
      float wd[8];
      int wq[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const lds_t* wb = w + 34 * min(b0 + u, nblk - 1);
        wd[u] = (float)__builtin_bit_cast(_Float16, lds_load<unsigned short>(wb));
        wq[u] = (int)((unsigned)lds_load<unsigned short>(wb + 2 + 4 * l) |
                      ((unsigned)lds_load<unsigned short>(wb + 4 + 4 * l) << 16));
      }
#pragma unroll
      for (int c = 0; c < MC; ++c) {
        if (MC == 1 || c < nc) {
          float ad[8];
          int aq[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int bb = min(b0 + u, nblk - 1);
            ad[u] = lds_load<float>(act - 4 - 4 * l + c * abytes + 36 * bb);
            aq[u] = lds_load<int>(act + c * abytes + 36 * bb);
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float r = __builtin_fmaf((float)__builtin_amdgcn_sdot4(wq[u], aq[u], 0, false),
                                           wd[u] * ad[u], acc[c]);
            acc[c] = b0 + u < nblk ? r : acc[c];
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < MC; ++c) {
      if (MC == 1 || c < nc) {
        float s = q8_hsum8(acc[c], threadIdx.x);
        if (live && l == 0) {
          if (p.add) s = s + (MC == 1 ? addv : gload<float>(p.add + row * p.add_nb0 + (c0 + c) * p.add_nb1));
          gstore<float>(p.dst + q8_unperm_row(row, p.perm_hd, p.perm_rows) * p.dst_nb0 + (c0 + c) * p.dst_nb1, s);
        }
      }
    }
  }
}

// The staged form for one column (a decode step's long rows, e.g. the FFN
// down projection): kQ8S1Waves waves per 8-row group. The waves request the
// group's rows and the column's blocks into LDS together; then each wave
// forms the operands of one slice of the blocks -- float(int8 dot) and
// fp16(w.d) * a.d per (block, lane), exactly the staged form's -- into LDS,
// and wave 0 runs each lane's chain of multiply-adds over the blocks in order.
// The same operations in the same order as the staged form, spread over the
// workgroup: a single wave's operand work (5 LDS reads and ~12 vector
// instructions per block) was the launch's longest phase.
constexpr int kQ8S1Waves = 8;
constexpr int kQ8S1LdsMax = 150 * 1024;

// LDS of the one-column staged form: rows, the column's blocks (each region
// whole 1 KB transfers), the operands.
__host__ __device__ inline int64_t q8_s1_lds_bytes(int64_t w_nb1, int64_t k) {
  return round1k(8 * w_nb1) + round1k(k / 32 * 36) + (k / 32) * kWave * 8;
}

__global__ __launch_bounds__(kQ8S1Waves * kWave) void mul_mat_q8_0_staged1_kernel(const Q8MulMat p) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) char stage_lds[];
  const lds_t* const lds = (const lds_t*)stage_lds;
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t g = blockIdx.x;
  const int nrows = (int)min<int64_t>(8, p.n - g * 8);
  const int64_t wbytes = (nrows - 1) * p.w_nb1 + p.k / 32 * 34;  // a multiple of 2
  const char* const wsrc = p.w + g * 8 * p.w_nb1;
  const int64_t wb4 = wbytes & ~int64_t(3);  // as in the staged form: a 2-byte tail is stored apart
  const int nblk = (int)(p.k / 32);
  const int abytes = nblk * 36;
  const int64_t act_off = round1k(8 * p.w_nb1);
  const int64_t op_off = act_off + round1k(abytes);
  {
    const rsrc_t r = make_rsrc(wsrc, (unsigned)wb4);
    const int n1k = (int)((wbytes + 1023) / 1024);
    for (int i = wv; i < n1k; i += kQ8S1Waves)
      dma16(r, (lds_t*)stage_lds + 1024 * i, (unsigned)(1024 * i + 16 * lane));
    const rsrc_t ra = make_rsrc(p.a, (unsigned)abytes);  // q8_s1_ok: 16-byte aligned, whole 16-byte groups
    for (int i = wv; i < (abytes + 1023) / 1024; i += kQ8S1Waves)
      dma16(ra, (lds_t*)stage_lds + act_off + 1024 * i, (unsigned)(1024 * i + 16 * lane));
  }
  const int l = lane & 7, r = lane >> 3;
  const int64_t row = g * 8 + r;
  const bool live = r < nrows;
  float addv = 0.0f;
  if (wv == 0 && p.add) addv = gload<float>(p.add + min(row, p.n - 1) * p.add_nb0);
  wait_vmem<0>();  // this wave's transfers (and the added term) have landed
  wg_barrier();
  if (wb4 != wbytes) {
    if (threadIdx.x == 0) lds_store<unsigned short>((lds_t*)(stage_lds + wb4), gload<unsigned short>(wsrc + wb4));
    wg_barrier();
  }
  // this wave's slice of the blocks: the operands of every (block, lane)
  const lds_t* const w = lds + (live ? r : 0) * p.w_nb1;
  const lds_t* const act = lds + act_off;
  lds_t* const op = (lds_t*)stage_lds + op_off;
  const int b_lo = nblk * wv / kQ8S1Waves, b_hi = nblk * (wv + 1) / kQ8S1Waves;
  for (int b = b_lo; b < b_hi; ++b) {
    const lds_t* wb = w + 34 * b;
    const float wd = (float)__builtin_bit_cast(_Float16, lds_load<unsigned short>(wb));
    const int wq = (int)((unsigned)lds_load<unsigned short>(wb + 2 + 4 * l) |
                         ((unsigned)lds_load<unsigned short>(wb + 4 + 4 * l) << 16));
    const float ad = lds_load<float>(act + 36 * b);
    const int aq = lds_load<int>(act + 36 * b + 4 + 4 * l);
    const f32x2_t o = {(float)__builtin_amdgcn_sdot4(wq, aq, 0, false), wd * ad};
    lds_store<f32x2_t>(op + 8 * (b * kWave + lane), o);
  }
  wg_barrier();
  if (wv != 0) return;
  // the chain, 8 blocks' operands read ahead of their multiply-adds
  float acc = 0.0f;
  int b0 = 0;
  for (; b0 + 8 <= nblk; b0 += 8) {
    f32x2_t o[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] = lds_load<f32x2_t>(op + 8 * ((b0 + u) * kWave + lane));
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(o[u].x, o[u].y, acc);
  }
  for (; b0 < nblk; ++b0) {
    const f32x2_t o = lds_load<f32x2_t>(op + 8 * (b0 * kWave + lane));
    acc = __builtin_fmaf(o.x, o.y, acc);
  }
  float s = q8_hsum8(acc, lane);
  if (live && l == 0) {
    if (p.add) s = s + addv;
    gstore<float>(p.dst + q8_unperm_row(row, p.perm_hd, p.perm_rows) * p.dst_nb0, s);
  }
}

// One column through the staged form's workgroup-wide variant: whole 16-byte
// groups of activation blocks at a 16-byte aligned address, and its LDS
// within the budget.
static bool q8_s1_ok(const Q8MulMat& p) {
  return p.m == 1 && !p.x && !p.swiglu_out && (p.k / 32 * 36) % 16 == 0 && reinterpret_cast<uintptr_t>(p.a) % 16 == 0 &&
         q8_s1_lds_bytes(p.w_nb1, p.k) <= kQ8S1LdsMax;
}

hipError_t launch_quantize_q8_0_act(const Q8Quantize& p, hipStream_t stream) {
  const int64_t n = p.rows * (p.ne0 / 32);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_q8_0_act_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     stream, p);
  return hipGetLastError();
}

bool q8_swiglu_out_ok(const Q8MulMat& p, int n_cu) {
  return p.swiglu_out && p.m == 1 && !p.add && !p.rope_on && !p.perm_hd && p.n % 64 == 0 &&
         p.n / 64 <= (n_cu > 0 ? n_cu : 256) && q8_ring_form(p);
}

bool q8_ring_form(const Q8MulMat& p) {
  const bool act_ok = p.x ? (p.x_ld >= p.k && reinterpret_cast<uintptr_t>(p.x) % 4 == 0)
                          : (p.a_nb1 % 4 == 0 && reinterpret_cast<uintptr_t>(p.a) % 4 == 0);
  // rows 4-byte aligned: every group's byte range ends on a whole dword (the
  // resource's range check is per dword)
  return p.w_nb1 <= kQ8RowBytesMax && p.k <= 960 && p.m <= kQ8Cols && (8 * p.w_nb1) % 16 == 0 &&
         p.w_nb1 % 4 == 0 &&
         reinterpret_cast<uintptr_t>(p.w) % 16 == 0 && act_ok && p.n * p.w_nb1 < (int64_t)1 << 40;
}

hipError_t launch_mul_mat_q8_0(const Q8MulMat& p, int n_cu, hipStream_t stream) {
  if (p.n == 0 || p.m == 0) return hipSuccess;
  const bool rows_form = q8_ring_form(p);
  if (p.x && !rows_form) return hipErrorInvalidValue;  // the prologue exists in the streaming form only
  if (rows_form) {
    typedef void (*ring_fn)(const Q8MulMat);
    static const ring_fn fns[2][kQ8Cols] = {
        {mul_mat_q8_0_ring_kernel<1, false>, mul_mat_q8_0_ring_kernel<2, false>, mul_mat_q8_0_ring_kernel<3, false>,
         mul_mat_q8_0_ring_kernel<4, false>, mul_mat_q8_0_ring_kernel<5, false>, mul_mat_q8_0_ring_kernel<6, false>,
         mul_mat_q8_0_ring_kernel<7, false>, mul_mat_q8_0_ring_kernel<8, false>},
        {mul_mat_q8_0_ring_kernel<1, true>, mul_mat_q8_0_ring_kernel<2, true>, mul_mat_q8_0_ring_kernel<3, true>,
         mul_mat_q8_0_ring_kernel<4, true>, mul_mat_q8_0_ring_kernel<5, true>, mul_mat_q8_0_ring_kernel<6, true>,
         mul_mat_q8_0_ring_kernel<7, true>, mul_mat_q8_0_ring_kernel<8, true>}};
    static const hipError_t attr = [] {
      hipError_t e = hipSuccess;
      for (int v = 0; v < 2; ++v)
        for (int m = 0; m < kQ8Cols; ++m)
          if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)fns[v][m], hipFuncAttributeMaxDynamicSharedMemorySize, kQ8RingLdsAll);
      return e;
    }();
    if (attr != hipSuccess) return attr;
    const int64_t groups = (p.n + 7) / 8;
    if (p.swiglu_out && !q8_swiglu_out_ok(p, n_cu)) return hipErrorInvalidValue;
    // with the SwiGLU epilogue one workgroup per 64-row block (8 groups)
    const unsigned grid = p.swiglu_out ? (unsigned)(p.n / 64)
                                       : (unsigned)std::min<int64_t>(n_cu > 0 ? n_cu : 256,
                                                                     (groups + kQ8RingWaves - 1) / kQ8RingWaves);
    const bool epi = p.rope_on || p.perm_hd;
    hipLaunchKernelGGL(fns[epi ? 1 : 0][p.m - 1], dim3(grid), dim3(kQ8RingWaves * kWave), kQ8RingLdsAll, stream, p);
  } else if (q8_stage_lds_bytes(p.w_nb1, p.k) <= kQ8StageLdsMax &&
             reinterpret_cast<uintptr_t>(p.w) % 16 == 0 && (8 * p.w_nb1) % 16 == 0 &&
             p.a_nb1 % 4 == 0 && reinterpret_cast<uintptr_t>(p.a) % 4 == 0) {
    static const hipError_t attr = [] {
      hipError_t e = hipSuccess;
      const void* fns[2] = {(const void*)&mul_mat_q8_0_staged_kernel<1>,
                            (const void*)&mul_mat_q8_0_staged_kernel<kQ8Cols>};
      for (const void* f : fns)
        if (e == hipSuccess) e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kQ8StageLdsMax);
      return e;
    }();
    if (attr != hipSuccess) return attr;
    const dim3 grid((unsigned)((p.n + 7) / 8));
    if (q8_s1_ok(p)) {
      static const hipError_t attr1 = hipFuncSetAttribute((const void*)&mul_mat_q8_0_staged1_kernel,
                                                          hipFuncAttributeMaxDynamicSharedMemorySize, kQ8S1LdsMax);
      if (attr1 != hipSuccess) return attr1;
      hipLaunchKernelGGL(mul_mat_q8_0_staged1_kernel, grid, dim3(kQ8S1Waves * kWave),
                         (unsigned)q8_s1_lds_bytes(p.w_nb1, p.k), stream, p);
      return hipGetLastError();
    }
    const unsigned lds = (unsigned)q8_stage_lds_bytes(p.w_nb1, p.k);
    if (p.m == 1)
      hipLaunchKernelGGL(mul_mat_q8_0_staged_kernel<1>, grid, dim3(kWave), lds, stream, p);
    else
      hipLaunchKernelGGL(mul_mat_q8_0_staged_kernel<kQ8Cols>, grid, dim3(kWave), lds, stream, p);
  } else {
    hipLaunchKernelGGL(mul_mat_q8_0_kernel, dim3((unsigned)((p.n + 31) / 32)), dim3(256), 0, stream,
                       p);
  }
  return hipGetLastError();
}

}  // namespace mi
