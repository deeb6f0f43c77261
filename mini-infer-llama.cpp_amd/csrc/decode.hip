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
// The wave's G query vectors stay in registers for the whole kernel, spread
// over the 16 lanes of each row. Per 64-position tile, one wave:
//   1. requests the tile's K rows (coalesced 16-byte loads);
//   2. stages K rows 64 dims at a time through a swizzled LDS tile and lets
//      lane i own position i: each lane dots its row with the G queries, whose
//      elements reach every lane as DPP row-broadcast FMA operands;
//   3. requests the tile's V rows, updates the running max (DPP row
//      reduction + readlane, no LDS),
//      rescales, exponentiates (exp2 of log2e-prescaled scores) and writes
//      the probabilities to LDS;
//   4. accumulates P.V with lanes owning 4 output dims of one row.
// Waves of a workgroup merge through LDS. With one split the workgroup writes
// the output; otherwise it writes an (m, l, acc) record per head to the
// workspace and decode_merge_kernel, launched next on the same stream,
// combines the splits with the stable rescaling
// O = sum_s 2^(m_s - M) A_s / sum_s 2^(m_s - M) L_s.
// (No cross-workgroup signalling inside a kernel: on this part a device-scope
// fence writes back and invalidates the whole L2 of the XCD.)
#include <cstdlib>

#include "attn_common.h"
#include "kernels.h"

namespace mi {

template <int D, typename KT, int G>
__device__ __forceinline__ void decode_body(const DecodeParams& p) {
  constexpr int ELT = (int)sizeof(KT);
  constexpr int NCH = D / 64;                    // 64-dim chunks staged for QK
  constexpr int LPR = D / 4;                     // PV: lanes per cache row
  constexpr int RPI = kWave / LPR;               // PV: rows per load instruction
  constexpr int NV = kDecodeTile / RPI;          // PV: load instructions per tile
  constexpr int TS = kDecodeTile * 64;  // LDS floats per wave (swizzled, unpadded)
  constexpr int HDR = (2 * G + 3) & ~3;          // record header: m[G], l[G]
  constexpr int REC = HDR + G * D;               // one merge record

  extern __shared__ float lds[];

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

  // The G query vectors, spread over the 16 lanes of every row:
  // qv[h][c] = Q[head0 + h][16 c + (lane & 15)]. A DPP row broadcast hands
  // dim 16 c + j to every lane as an FMA operand: no memory round trip.
  float qv[G][D / 16];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int c = 0; c < D / 16; ++c) qv[h][c] = q0[h * q_s1f + 16 * c + (lane & 15)];

  for (int p0 = lo + wave * kDecodeTile; p0 < hi; p0 += nwaves * kDecodeTile) {
    const int nvalid = min(kDecodeTile, hi - p0);
    const int last = nvalid - 1;
    const char* ktile = kbase + (int64_t)p0 * it.k_s2;  // wave-uniform
    const char* vtile = vbase + (int64_t)p0 * it.v_s2;

    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = 0.f;
    float4 vreg[NV];

#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      // Rows p0..p0+63, dims [64c, 64c+64) of KV head g: row r is 256
      // contiguous LDS bytes whose 16-byte slot s holds chunk s ^ (r & 15),
      // so lane r reading chunk d of its own row hits 16 distinct bank groups
      // across 16 lanes. Rows past the split end re-read its last row (their
      // scores are masked).
      float4 kreg[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const unsigned off = (unsigned)(min(i * 4 + kr, last) * ks2 + (c * 64 + kc * 4) * ELT);
        kreg[i] = load4<KT>(ktile + off);
      }
      wave_lds_fence();
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = i * 4 + kr;
        *reinterpret_cast<float4*>(&klds[row * 64 + ((kc ^ (row & 15)) * 4)]) = kreg[i];
      }
      wave_lds_fence();

      // Lane = position: dot its row with the G queries. (qv passes through an
      // empty asm so the broadcasts stay here instead of being hoisted out of
      // the tile loop, which would need one register per broadcast value.)
#pragma unroll
      for (int q16 = 0; q16 < 4; ++q16) {
#pragma unroll
        for (int h = 0; h < G; ++h) asm volatile("" : "+v"(qv[h][c * 4 + q16]));
        const float4 k0 = *reinterpret_cast<const float4*>(
            &klds[lane * 64 + (((4 * q16 + 0) ^ (lane & 15)) * 4)]);
        const float4 k1 = *reinterpret_cast<const float4*>(
            &klds[lane * 64 + (((4 * q16 + 1) ^ (lane & 15)) * 4)]);
        const float4 k2 = *reinterpret_cast<const float4*>(
            &klds[lane * 64 + (((4 * q16 + 2) ^ (lane & 15)) * 4)]);
        const float4 k3 = *reinterpret_cast<const float4*>(
            &klds[lane * 64 + (((4 * q16 + 3) ^ (lane & 15)) * 4)]);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float qq = qv[h][c * 4 + q16];
          float a = s[h];
          a = fmac_bcast<0>(a, qq, k0.x);
          a = fmac_bcast<1>(a, qq, k0.y);
          a = fmac_bcast<2>(a, qq, k0.z);
          a = fmac_bcast<3>(a, qq, k0.w);
          a = fmac_bcast<4>(a, qq, k1.x);
          a = fmac_bcast<5>(a, qq, k1.y);
          a = fmac_bcast<6>(a, qq, k1.z);
          a = fmac_bcast<7>(a, qq, k1.w);
          a = fmac_bcast<8>(a, qq, k2.x);
          a = fmac_bcast<9>(a, qq, k2.y);
          a = fmac_bcast<10>(a, qq, k2.z);
          a = fmac_bcast<11>(a, qq, k2.w);
          a = fmac_bcast<12>(a, qq, k3.x);
          a = fmac_bcast<13>(a, qq, k3.y);
          a = fmac_bcast<14>(a, qq, k3.z);
          a = fmac_bcast<15>(a, qq, k3.w);
          s[h] = a;
        }
      }
    }

    // V rows of the tile (requested after QK so that the V and K register
    // sets never coexist; other waves cover the latency).
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int row = i * RPI + vr;
      const unsigned off = (unsigned)(min(row, last) * vs2 + vc * 4 * ELT);
      const float4 x = load4<KT>(vtile + off);
      vreg[i] = row < nvalid ? x : zero4;
    }

    // Online softmax: wave-uniform running max per head (DPP + readlane),
    // per-lane partial sums.
    const bool valid = lane < nvalid;
    float pv[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) pv[h] = 0.f;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float x = valid ? s[h] * p.scale_log2e : -INFINITY;
      const float mn = fmaxf(m[h], wave_max_dpp(x));
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
}

// Two occupancy variants of the same body: two waves per SIMD (register
// budget 256) or one (512).
template <int D, typename KT, int G>
__global__ __launch_bounds__(kDecodeWaves* kWave) __attribute__((amdgpu_waves_per_eu(2)))
void decode_kernel(const DecodeParams p) {
  decode_body<D, KT, G>(p);
}

template <int D, typename KT, int G>
__global__ __launch_bounds__(kDecodeWaves* kWave) void decode_kernel_wide(const DecodeParams p) {
  decode_body<D, KT, G>(p);
}

// Combines the split records of one (item, head chunk) per workgroup in two
// passes: per head the max m over splits, the weights w_s = 2^(m_s - m) and
// the denominator; then every (head, dim) output is an independent weighted
// sum over the splits' unnormalised accumulators.
template <int D, int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(const DecodeParams p) {
  constexpr int HDR = (2 * G + 3) & ~3;
  constexpr int REC = HDR + G * D;
  extern __shared__ float lds[];  // w[G][splits], inv_l[G]
  const int grp = blockIdx.x;
  const int per_item = p.n_head_kv * p.n_chunks;
  const DecodeItem& it = p.item[grp / per_item];
  const int g = (grp % per_item) / p.n_chunks;
  const int hc = grp % p.n_chunks;
  const int head0 = g * p.n_rep + hc * G;
  const int S = p.splits;
  const float* base = p.part + (int64_t)grp * S * REC;
  float* w = lds;
  float* inv_l = lds + G * S;

  // pass 1: one wave per head (round robin), lanes over splits
  const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
  for (int h = wv; h < G; h += blockDim.x / kWave) {
    float mx = -INFINITY;
    for (int sp = lane; sp < S; sp += kWave) mx = fmaxf(mx, base[(int64_t)sp * REC + h]);
    mx = wave_max_dpp(mx);
    float den = 0.f;
    for (int sp = lane; sp < S; sp += kWave) {
      const float* r = base + (int64_t)sp * REC;
      const float wt = fast_exp2(r[h] - mx);  // empty split: m = -inf -> 0
      w[h * S + sp] = wt;
      den += wt * r[G + h];
    }
    den = wave_sum(den);
    if (lane == 0) inv_l[h] = 1.f / den;
  }
  __syncthreads();

  // pass 2: independent weighted sums
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int h = idx / D, d = idx % D;
    const float* a = base + HDR + h * D + d;
    const float* wh = w + h * S;
    // 8 independent loads per round keep the split records' latency overlapped.
    float acc8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int sp = 0;
    for (; sp + 8 <= S; sp += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) acc8[u] = fmaf(wh[sp + u], a[(int64_t)(sp + u) * REC], acc8[u]);
    }
    for (; sp < S; ++sp) acc8[0] = fmaf(wh[sp], a[(int64_t)sp * REC], acc8[0]);
    float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it.out) +
                                        (int64_t)(head0 + h) * it.o_s1);
    o[d] = (((acc8[0] + acc8[1]) + (acc8[2] + acc8[3])) + ((acc8[4] + acc8[5]) + (acc8[6] + acc8[7]))) *
           inv_l[h];
  }
}

template <int D, typename KT, int G>
static hipError_t launch_decode_t(const DecodeParams& p, hipStream_t stream) {
  const size_t lds_max = (size_t)kDecodeWaves * kDecodeTile * 64 * sizeof(float);
  // head_dim 64: two waves per SIMD unless MI_HIP_DECODE_WIDE=1; head_dim 128: one.
  static const bool wide = D > 64 || [] {
    const char* e = std::getenv("MI_HIP_DECODE_WIDE");
    return e && e[0] == '1';
  }();
  const void* fn = wide ? reinterpret_cast<const void*>(&decode_kernel_wide<D, KT, G>)
                        : reinterpret_cast<const void*>(&decode_kernel<D, KT, G>);
  static const hipError_t attr = hipFuncSetAttribute(
      fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max);
  if (attr != hipSuccess) return attr;
  const unsigned groups = (unsigned)(p.n_items * p.n_head_kv * p.n_chunks);
  const size_t lds = (size_t)p.waves * kDecodeTile * 64 * sizeof(float);
  if (wide)
    hipLaunchKernelGGL((decode_kernel_wide<D, KT, G>), dim3((unsigned)p.splits, groups),
                       dim3(p.waves * kWave), lds, stream, p);
  else
    hipLaunchKernelGGL((decode_kernel<D, KT, G>), dim3((unsigned)p.splits, groups),
                       dim3(p.waves * kWave), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  hipLaunchKernelGGL((decode_merge_kernel<D, G>), dim3(groups), dim3(256),
                     ((size_t)G * p.splits + G) * sizeof(float), stream, p);
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
