// decode.hip -- fused ATTN_QK -> causal SOFTMAX -> ATTN_KQV for one query
// token (src/ops_cpu.cpp:304-410 with n_tokens == 1), HBM-bound, no MFMA.
//
// Work decomposition
//   grid.y = (item, KV head g, head chunk): the G Q heads g*n_rep + hc*G ..
//            + G - 1 that share KV head g (GQA is an index mapping: every
//            K/V row is read once for all G heads, never copied).
//   grid.x = split of the positions [0, n_kv) (split-KV); each workgroup's
//            kDecodeWaves waves take interleaved 64-position tiles of its
//            split and keep a running (max, sum, acc) per head.
// Per 64-position tile, one wave:
//   1. streams the tile's V rows into registers (coalesced 16-byte loads,
//      D/4 lanes per row) so their latency overlaps the QK work;
//   2. stages K rows 64 dims at a time through a padded LDS tile and then
//      lets lane i own position i: each lane dots its row with the G query
//      vectors, which are wave-uniform and read through the scalar cache;
//   3. updates the running max with a wave reduction, rescales, exponentiates
//      (exp2 of log2e-prescaled scores) and writes the probabilities to LDS;
//   4. accumulates P.V with lanes owning 4 output dims of one row.
// Waves of a workgroup merge through LDS; splits merge through a workspace:
// the last workgroup of an (item, head chunk) to arrive (device-scope
// counter) combines all split partials with the stable rescaling
// O = sum_s 2^(m_s - M) A_s / sum_s 2^(m_s - M) L_s and resets the counter.
#include "attn_common.h"
#include "kernels.h"

namespace mi {

// One 16-byte LDS slot per lane of the K tile (lane l of the instruction
// whose wave-uniform base is `dst` lands at dst + 4*l floats).
template <typename KT>
__device__ inline void stage_k_slot(const char* src, float* dst, int lane);

// F32 cache: direct global -> LDS transfer, no register staging.
template <>
__device__ inline void stage_k_slot<float>(const char* src, float* dst, int lane) {
  (void)lane;
  __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src),
                                   (__attribute__((address_space(3))) void*)(dst),
                                   16, 0, 0);
}

// F16 cache: 8-byte load, exact widening, 16-byte LDS store.
template <>
__device__ inline void stage_k_slot<_Float16>(const char* src, float* dst, int lane) {
  *reinterpret_cast<float4*>(dst + 4 * lane) = load4<_Float16>(src);
}

// (The compiler's wait-count pass tracks the direct-to-LDS transfers and
// waits for them before the first LDS read of the tile.)

// qa[h][0..3] = Q[head0 + h][4*step .. 4*step+3] through the scalar cache.
template <int G>
__device__ inline void load_q4(float (&qa)[G][4], const float* qrow, int64_t q_s1f, int step) {
  const const_f32_ptr qc = as_const(qrow);
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 4; ++e) qa[h][e] = qc[h * q_s1f + step * 4 + e];
}

template <int D, typename KT, int G>
__global__ __launch_bounds__(kDecodeWaves* kWave) void decode_kernel(const DecodeParams p) {
  constexpr int ELT = (int)sizeof(KT);
  constexpr int NCH = D / 64;                    // 64-dim chunks staged for QK
  constexpr int LPR = D / 4;                     // PV: lanes per cache row
  constexpr int RPI = kWave / LPR;               // PV: rows per load instruction
  constexpr int NV = kDecodeTile / RPI;          // PV: load instructions per tile
  constexpr int NV0 = NV < 16 ? NV : 16;         // of which issued before QK
  constexpr int TS = kDecodeTile * 64;  // LDS floats per wave (swizzled, unpadded)
  constexpr int HDR = (2 * G + 3) & ~3;          // record header: m[G], l[G]
  constexpr int REC = HDR + G * D;               // one merge record

  extern __shared__ float lds[];
  __shared__ int s_last;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;

  const int split = blockIdx.x;
  const int grp = blockIdx.y;
  const int per_item = p.n_head_kv * p.n_chunks;
  const int it_idx = grp / per_item;
  const int g = (grp % per_item) / p.n_chunks;
  const int hc = grp % p.n_chunks;
  const DecodeItem& it = p.item[it_idx];

  const int n_kv = it.n_kv;
  const int per_split =
      ((n_kv + p.splits - 1) / p.splits + kDecodeTile - 1) / kDecodeTile * kDecodeTile;
  const int lo = split * per_split;
  const int hi = min(n_kv, lo + per_split);
  const int head0 = g * p.n_rep + hc * G;

  const char* kbase = it.k + (int64_t)g * it.k_s1;
  const char* vbase = it.v + (int64_t)g * it.v_s1;
  const float* q0 = reinterpret_cast<const float*>(reinterpret_cast<const char*>(it.q) +
                                                   (int64_t)head0 * it.q_s1);
  const int64_t q_s1f = it.q_s1 / 4;

  float* klds = lds + wave * TS;

  float m[G], l[G], acc[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[h][e] = 0.f;
  }

  const int kr = lane >> 4, kc = lane & 15;    // K staging: 16 lanes per 64-dim row
  const int vr = lane / LPR, vc = lane % LPR;  // PV: LPR lanes per row
  // Strides fit 32 bits (checked by the host: 64 rows of any stride < 2^31).
  const int ks2 = (int)it.k_s2, vs2 = (int)it.v_s2;
  const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);

  for (int p0 = lo + wave * kDecodeTile; p0 < hi; p0 += nwaves * kDecodeTile) {
    const int nvalid = min(kDecodeTile, hi - p0);
    const int last = nvalid - 1;
    const char* ktile = kbase + (int64_t)p0 * it.k_s2;  // wave-uniform
    const char* vtile = vbase + (int64_t)p0 * it.v_s2;

    float4 vreg[NV];
    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = 0.f;

#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      // Stage rows p0..p0+63, dims [64c, 64c+64) of KV head g into the wave's
      // LDS tile. Row r is 256 contiguous bytes; its 16-byte slot s holds the
      // row's chunk s ^ (r & 15), so lane r reading chunk d4 of its own row
      // (slot d4 ^ (r & 15)) hits 16 distinct bank groups across 16 lanes.
      // Rows past the split end re-read its last row (their scores are masked).
      wave_lds_fence();
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = i * 4 + kr;
        const unsigned off =
            (unsigned)(min(row, last) * ks2 + (c * 64 + ((kc ^ (row & 15)) * 4)) * ELT);
        stage_k_slot<KT>(ktile + off, klds + i * 256, lane);
      }
      // Keep every K transfer ahead of the V loads in issue order, so that
      // waiting for K leaves the V loads in flight.
      asm volatile("" ::: "memory");
      if (c == 0) {
        // V rows of the tile: in flight during the QK work.
#pragma unroll
        for (int i = 0; i < NV0; ++i) {
          const int row = i * RPI + vr;
          const unsigned off = (unsigned)(min(row, last) * vs2 + vc * 4 * ELT);
          const float4 x = load4<KT>(vtile + off);
          vreg[i] = row < nvalid ? x : zero4;
        }
      }
      wave_lds_fence();

      // Q for this chunk is wave-uniform: scalar loads, pipelined one
      // 4-dim step ahead through a pointer the compiler may not hoist.
      const float* qrow = q0 + c * 64;
      float qa[G][4], qn[G][4];
      load_q4<G>(qa, qrow, q_s1f, 0);
#pragma unroll
      for (int d4 = 0; d4 < 16; ++d4) {
        if (d4 + 1 < 16) {
          asm volatile("" : "+s"(qrow));
          load_q4<G>(qn, qrow, q_s1f, d4 + 1);
        }
        const float4 kv = *reinterpret_cast<const float4*>(
            &klds[lane * 64 + ((d4 ^ (lane & 15)) * 4)]);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          s[h] = fmaf(kv.x, qa[h][0], s[h]);
          s[h] = fmaf(kv.y, qa[h][1], s[h]);
          s[h] = fmaf(kv.z, qa[h][2], s[h]);
          s[h] = fmaf(kv.w, qa[h][3], s[h]);
        }
        if (d4 + 1 < 16) {
#pragma unroll
          for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) qa[h][e] = qn[h][e];
        }
      }
    }

    // Online softmax: wave-uniform running max per head, per-lane partial sums.
    const bool valid = lane < nvalid;
    float pv[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) pv[h] = 0.f;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float x = valid ? s[h] * p.scale_log2e : -INFINITY;
      const float mn = fmaxf(m[h], wave_max(x));
      const float alpha = fast_exp2(m[h] - mn);
      const float e = fast_exp2(x - mn);
      l[h] = l[h] * alpha + e;
      m[h] = mn;
      pv[h] = e;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[h][j] *= alpha;
    }

    // Probabilities to LDS, [row][8], over the (now dead) K tile.
    wave_lds_fence();
    *reinterpret_cast<float4*>(&klds[lane * 8]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
    if (G > 4)
      *reinterpret_cast<float4*>(&klds[lane * 8 + 4]) = make_float4(pv[4], pv[5], pv[6], pv[7]);
    wave_lds_fence();

#pragma unroll
    for (int i = NV0; i < NV; ++i) {
      const int row = i * RPI + vr;
      const unsigned off = (unsigned)(min(row, last) * vs2 + vc * 4 * ELT);
      const float4 x = load4<KT>(vtile + off);
      vreg[i] = row < nvalid ? x : zero4;
    }

#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int row = i * RPI + vr;
      const float4 pa = *reinterpret_cast<const float4*>(&klds[row * 8]);
      float4 pb = zero4;
      if (G > 4) pb = *reinterpret_cast<const float4*>(&klds[row * 8 + 4]);
      const float pr[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
      const float4 vv = vreg[i];
#pragma unroll
      for (int h = 0; h < G; ++h) {
        acc[h][0] = fmaf(pr[h], vv.x, acc[h][0]);
        acc[h][1] = fmaf(pr[h], vv.y, acc[h][1]);
        acc[h][2] = fmaf(pr[h], vv.z, acc[h][2]);
        acc[h][3] = fmaf(pr[h], vv.w, acc[h][3]);
      }
    }
    wave_lds_fence();
  }

  // Wave totals: l over all lanes, acc over the RPI lanes sharing a column.
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] = wave_sum(l[h]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int off = LPR; off < kWave; off <<= 1) acc[h][j] += __shfl_xor(acc[h][j], off, kWave);
    }
  }

  // Workgroup merge through LDS.
  __syncthreads();
  float* rec = lds + wave * REC;
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      rec[h] = m[h];
      rec[G + h] = l[h];
    }
  }
  if (lane < LPR) {
#pragma unroll
    for (int h = 0; h < G; ++h)
      *reinterpret_cast<float4*>(&rec[HDR + h * D + 4 * lane]) =
          make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
  }
  __syncthreads();

  const bool direct = p.splits == 1;
  float* prec = p.part + ((int64_t)grp * p.splits + split) * REC;
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    float mx = -INFINITY;
    for (int w = 0; w < nwaves; ++w) mx = fmaxf(mx, lds[w * REC + h]);
    float a = 0.f, sum = 0.f;
    if (mx > -INFINITY) {
      for (int w = 0; w < nwaves; ++w) {
        const float sc = fast_exp2(lds[w * REC + h] - mx);
        a += sc * lds[w * REC + HDR + h * D + d];
        sum += sc * lds[w * REC + G + h];
      }
    }
    if (direct) {
      float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it.out) +
                                          (int64_t)(head0 + h) * it.o_s1);
      o[d] = a / sum;
    } else {
      prec[HDR + h * D + d] = a;
      if (d == 0) {
        prec[h] = mx;
        prec[G + h] = sum;
      }
    }
  }
  if (direct) return;

  // Split merge by the last workgroup to arrive.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(&p.counter[grp], 1u);
    s_last = prev == (unsigned)(p.splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* gbase = p.part + (int64_t)grp * p.splits * REC;
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    float mx = -INFINITY;
    for (int sp = 0; sp < p.splits; ++sp) mx = fmaxf(mx, gbase[sp * REC + h]);
    float a = 0.f, sum = 0.f;
    for (int sp = 0; sp < p.splits; ++sp) {
      const float* r = gbase + sp * REC;
      const float sc = fast_exp2(r[h] - mx);
      a += sc * r[HDR + h * D + d];
      sum += sc * r[G + h];
    }
    float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it.out) +
                                        (int64_t)(head0 + h) * it.o_s1);
    o[d] = a / sum;
  }
  if (threadIdx.x == 0) p.counter[grp] = 0u;
}

template <int D, typename KT, int G>
static hipError_t launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  const size_t lds = (size_t)kDecodeWaves * kDecodeTile * 64 * sizeof(float);
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&decode_kernel<D, KT, G>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (attr != hipSuccess) return attr;
  const dim3 grid((unsigned)p.splits, (unsigned)(p.n_items * p.n_head_kv * p.n_chunks));
  hipLaunchKernelGGL((decode_kernel<D, KT, G>), grid, dim3(kDecodeWaves * kWave), lds, stream, p);
  return hipGetLastError();
}

template <int D, typename KT>
static hipError_t launch_decode_g(const DecodeParams& p, int g, hipStream_t stream) {
  switch (g) {
    case 1: return launch_decode_t<D, KT, 1>(p, stream);
    case 2: return launch_decode_t<D, KT, 2>(p, stream);
    case 4: return launch_decode_t<D, KT, 4>(p, stream);
    case 7: return launch_decode_t<D, KT, 7>(p, stream);
    case 8: return launch_decode_t<D, KT, 8>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

int decode_group_size(int n_rep) {
  static const int kSizes[] = {8, 7, 4, 2, 1};
  for (int g : kSizes)
    if (n_rep % g == 0) return g;
  return 1;
}

size_t decode_record_floats(int head_dim, int group) {
  const int hdr = (2 * group + 3) & ~3;
  return (size_t)hdr + (size_t)group * head_dim;
}

hipError_t launch_decode(const DecodeParams& p, int head_dim, bool f16, int group,
                         hipStream_t stream) {
  if (head_dim == 64)
    return f16 ? launch_decode_g<64, _Float16>(p, group, stream)
               : launch_decode_g<64, float>(p, group, stream);
  if (head_dim == 128)
    return f16 ? launch_decode_g<128, _Float16>(p, group, stream)
               : launch_decode_g<128, float>(p, group, stream);
  return hipErrorInvalidValue;
}

}  // namespace mi
