// decode.hip -- fused ATTN_QK -> causal SOFTMAX -> ATTN_KQV for one query
// token (src/ops_cpu.cpp:304-410 with n_tokens == 1), HBM-bound, no MFMA.
//
// Work decomposition. A group is (item, KV head g, head chunk hc): the G Q
// heads g*n_rep + hc*G .. + G - 1 that read KV head g (GQA is an index
// mapping: every K/V row is read once for all G heads, never copied). A
// group's positions form ceil(n_kv / 64) tiles, split into nw contiguous runs,
// one per wave; each wave is a workgroup of its own. The host sizes nw so the
// launch has about one wave per SIMD and every run has the same number of
// tiles to within one.
//
// Per wave: the G query vectors stay in registers, spread over the 16 lanes of
// each row. The K and V tiles of NBUF tiles are requested up front and each
// slot is refilled as soon as its registers are free, so every wave keeps one
// to two tiles of HBM requests in flight while it computes. Loads go through
// buffer resources bounded by the group's last row: rows past n_kv read as
// zero without a memory request, and so do refills past the run's end (a
// zero-sized resource), which keeps the loop free of branches around loads.
// Per tile:
//   1. K rows go to a swizzled LDS tile and lane i takes position i: each
//      lane dots its row with the G queries, whose elements reach every lane
//      as DPP row-broadcast FMA operands (no memory round trip);
//   2. online softmax in base 2: running max by DPP row reduction + readlane,
//      exp2 of log2e-prescaled scores; probabilities to LDS;
//   3. P.V with lanes owning 4 output dims of one row, V straight from the
//      registers it was loaded into.
// A run that covers its whole group writes O; otherwise the wave writes an
// (m, l, acc) record and decode_merge_kernel, launched next on the same
// stream, combines the nw records of each group with the stable rescaling
// O = sum_s 2^(m_s - M) A_s / sum_s 2^(m_s - M) L_s.
// (No cross-workgroup signalling inside a kernel: on this part a device-scope
// fence writes back and invalidates the whole L2 of the XCD.)
#include <cstdlib>

#include "attn_common.h"
#include "kernels.h"

namespace mi {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw (unswizzled, stride 0) buffer descriptor word 3 of the gfx9 family.
constexpr int kRawBufferWord3 = 0x00020000;

// Descriptor over [p, p + bytes): loads at offsets >= bytes return zero and
// make no memory request.
__device__ inline rsrc_t make_rsrc(const char* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(p), (short)0, (int)bytes,
                                           kRawBufferWord3);
}

// Four consecutive cache elements, held in registers at storage width.
template <typename KT>
struct Cache;
template <>
struct Cache<float> {
  typedef f32x4 raw;
  static __device__ inline raw load(rsrc_t r, unsigned off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
  }
  static __device__ inline float4 widen(raw x) { return make_float4(x.x, x.y, x.z, x.w); }
};
template <>
struct Cache<_Float16> {
  typedef half4_t raw;
  static __device__ inline raw load(rsrc_t r, unsigned off) {
    return __builtin_bit_cast(half4_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
  }
  static __device__ inline float4 widen(raw h) {
    return make_float4((float)h.x, (float)h.y, (float)h.z, (float)h.w);
  }
};

// Record of one wave's run: m[G], l[G] (padded to 4), then acc[G][D].
__host__ __device__ constexpr int record_header(int g) { return (2 * g + 3) & ~3; }

// s[J % NACC][h] += bcast_J(q[h]) * k for all heads; heads are interleaved so
// the DPP operand of an instruction was written at least two instructions
// earlier (no hazard wait states).
template <int J, int G, int NACC>
__device__ __forceinline__ void qk_step(float (&s)[NACC][G], const float (&q)[G], float k) {
#pragma unroll
  for (int h = 0; h < G; ++h) s[J % NACC][h] = fmac_bcast<J>(s[J % NACC][h], q[h], k);
}

// DEPTH: tiles of K/V requested ahead per wave. Depth 1 keeps the wave within
// 256 registers, so each SIMD runs two waves and one computes while the other
// waits on memory; depth 2 holds two tiles (one wave per SIMD).
template <int D, typename KT, int G, int DEPTH>
__device__ __forceinline__ void decode_body(const DecodeParams& p) {
  typedef Cache<KT> C;
  typedef typename C::raw raw_t;
  constexpr int ELT = (int)sizeof(KT);
  constexpr int NCH = D / 64;                 // 64-dim K chunks per row
  constexpr int NK = NCH * 16;                // K loads per lane per tile
  constexpr int LPR = D / 4;                  // PV: lanes per V row
  constexpr int RPI = kWave / LPR;            // PV: rows per load
  constexpr int NV = kDecodeTile / RPI;       // V loads per lane per tile
  constexpr int NBUF = DEPTH;
  constexpr int NACC = G >= 3 ? 1 : (G == 2 ? 2 : 3);
  constexpr int HDR = record_header(G);
  constexpr int REC = HDR + G * D;
  constexpr int CS = kDecodeTile * 64;        // LDS floats per staged K chunk

  __shared__ float klds[NCH * CS];  // the K tile (F32, swizzled), then P

  const int lane = threadIdx.x;
  const int wid = blockIdx.x;

  // item, group and run of this wave (items are few: a scalar scan)
  int ii = 0;
  while (ii + 1 < p.n_items && wid >= p.item[ii + 1].wave0) ++ii;
  const DecodeItem& it = p.item[ii];
  const int local = wid - it.wave0;
  const int gl = local / it.nw;
  const int run = local - gl * it.nw;
  const int g = gl / p.n_chunks;
  const int hc = gl - g * p.n_chunks;
  const int head0 = g * p.n_rep + hc * G;
  const int n_kv = it.n_kv;
  const int tpg = (n_kv + kDecodeTile - 1) / kDecodeTile;
  const int t_begin = (int)((int64_t)tpg * run / it.nw);
  const int t_end = (int)((int64_t)tpg * (run + 1) / it.nw);

  // Offsets are 32-bit (the host checks n_kv * stride < 2^31).
  const int ks2 = (int)it.k_s2, vs2 = (int)it.v_s2;
  const rsrc_t kres = make_rsrc(it.k + (int64_t)g * it.k_s1, (unsigned)((n_kv - 1) * ks2 + D * ELT));
  const rsrc_t vres = make_rsrc(it.v + (int64_t)g * it.v_s1, (unsigned)((n_kv - 1) * vs2 + D * ELT));
  const rsrc_t none = make_rsrc(it.k, 0u);

  const int kr = lane >> 4, kc = lane & 15;    // K staging: 16 lanes per 64-dim chunk row
  const int vr = lane / LPR, vc = lane % LPR;  // PV: LPR lanes per V row
  const unsigned klane = (unsigned)(kr * ks2 + kc * 4 * ELT);
  const unsigned vlane = (unsigned)(vr * vs2 + vc * 4 * ELT);

  // The G query vectors, requested before any cache tile:
  // qv[h][c] = Q[head0 + h][16 c + (lane & 15)].
  float qv[G][D / 16];
  {
    const float* q0 = reinterpret_cast<const float*>(reinterpret_cast<const char*>(it.q) +
                                                     (int64_t)head0 * it.q_s1);
    const int64_t q_s1f = it.q_s1 / 4;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int c = 0; c < D / 16; ++c) qv[h][c] = q0[h * q_s1f + 16 * c + (lane & 15)];
  }

  raw_t kb[NBUF][NK], vb[NBUF][NV];
  // (the lane's base offset passes through an empty asm at every issue so the
  // per-load offsets are formed next to their loads instead of being hoisted
  // out of the loop, which would hold one register per load)
  auto issue_k = [&](raw_t (&dst)[NK], int t) __attribute__((always_inline)) {
    const rsrc_t r = t < t_end ? kres : none;
    unsigned base = klane;
    asm volatile("" : "+v"(base));
    base += (unsigned)(t * kDecodeTile * ks2);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        dst[c * 16 + i] = C::load(r, base + (unsigned)(i * 4 * ks2 + c * 64 * ELT));
  };
  auto issue_v = [&](raw_t (&dst)[NV], int t) __attribute__((always_inline)) {
    const rsrc_t r = t < t_end ? vres : none;
    unsigned base = vlane;
    asm volatile("" : "+v"(base));
    base += (unsigned)(t * kDecodeTile * vs2);
#pragma unroll
    for (int i = 0; i < NV; ++i) dst[i] = C::load(r, base + (unsigned)(i * RPI * vs2));
  };
#pragma unroll
  for (int b = 0; b < NBUF; ++b) {
    issue_k(kb[b], t_begin + b);
    issue_v(vb[b], t_begin + b);
  }

  float m[G], l[G], acc[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[h][e] = 0.f;
  }

  auto process = [&](raw_t (&kt)[NK], raw_t (&vt)[NV], int t) __attribute__((always_inline)) {
    const int nvalid = min(kDecodeTile, n_kv - t * kDecodeTile);

    // K tile to LDS: chunk c of row r is 256 contiguous bytes whose 16-byte
    // slot s holds dims 64c + 4 (s ^ (r & 15)) .. +3, so lane r reading slot
    // d of its own row hits 16 distinct bank groups across 16 lanes.
    wave_lds_fence();
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = i * 4 + kr;
        *reinterpret_cast<float4*>(&klds[c * CS + row * 64 + ((kc ^ (row & 15)) * 4)]) =
            C::widen(kt[c * 16 + i]);
      }
    wave_lds_fence();
    issue_k(kt, t + NBUF);  // the slot's K registers are free again

    float s[NACC][G];
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
      for (int h = 0; h < G; ++h) s[a][h] = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const float* krow = klds + c * CS + lane * 64;
#pragma unroll
      for (int q16 = 0; q16 < 4; ++q16) {
        // (qv passes through an empty asm so the broadcasts stay here instead
        // of being hoisted out of the tile loop, which would need one
        // register per broadcast value)
        float qq[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
          asm volatile("" : "+v"(qv[h][c * 4 + q16]));
          qq[h] = qv[h][c * 4 + q16];
        }
        const float4 k0 = *reinterpret_cast<const float4*>(&krow[((4 * q16 + 0) ^ (lane & 15)) * 4]);
        const float4 k1 = *reinterpret_cast<const float4*>(&krow[((4 * q16 + 1) ^ (lane & 15)) * 4]);
        const float4 k2 = *reinterpret_cast<const float4*>(&krow[((4 * q16 + 2) ^ (lane & 15)) * 4]);
        const float4 k3 = *reinterpret_cast<const float4*>(&krow[((4 * q16 + 3) ^ (lane & 15)) * 4]);
        qk_step<0>(s, qq, k0.x);
        qk_step<1>(s, qq, k0.y);
        qk_step<2>(s, qq, k0.z);
        qk_step<3>(s, qq, k0.w);
        qk_step<4>(s, qq, k1.x);
        qk_step<5>(s, qq, k1.y);
        qk_step<6>(s, qq, k1.z);
        qk_step<7>(s, qq, k1.w);
        qk_step<8>(s, qq, k2.x);
        qk_step<9>(s, qq, k2.y);
        qk_step<10>(s, qq, k2.z);
        qk_step<11>(s, qq, k2.w);
        qk_step<12>(s, qq, k3.x);
        qk_step<13>(s, qq, k3.y);
        qk_step<14>(s, qq, k3.z);
        qk_step<15>(s, qq, k3.w);
      }
    }

    // Online softmax: wave-uniform running max per head, per-lane sums.
    const bool valid = lane < nvalid;
    float pv[8];
#pragma unroll
    for (int h = 0; h < 8; ++h) pv[h] = 0.f;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float sh = s[0][h];
#pragma unroll
      for (int a = 1; a < NACC; ++a) sh += s[a][h];
      const float x = valid ? sh * p.scale_log2e : -INFINITY;
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

    // O += P.V (rows past n_kv loaded as zero and have P = 0).
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int row = i * RPI + vr;
      const float4 pa = *reinterpret_cast<const float4*>(&klds[row * 8]);
      float4 pb = make_float4(0.f, 0.f, 0.f, 0.f);
      if (G > 4) pb = *reinterpret_cast<const float4*>(&klds[row * 8 + 4]);
      const float pr[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
      const float4 vv = C::widen(vt[i]);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        acc[h][0] = fmaf(pr[h], vv.x, acc[h][0]);
        acc[h][1] = fmaf(pr[h], vv.y, acc[h][1]);
        acc[h][2] = fmaf(pr[h], vv.z, acc[h][2]);
        acc[h][3] = fmaf(pr[h], vv.w, acc[h][3]);
      }
    }
    issue_v(vt, t + NBUF);
  };

  // Slots are used in turn; exits leave the loop rather than re-entering it,
  // so the wait counts at the loop head see one pattern of loads in flight.
  int t = t_begin;
  while (true) {
    process(kb[0], vb[0], t);
    if (++t >= t_end) break;
    if (NBUF > 1) {
      process(kb[NBUF - 1], vb[NBUF - 1], t);
      if (++t >= t_end) break;
    }
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

  if (it.nw == 1) {  // the run is the whole group
    if (lane < LPR) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float inv = 1.f / l[h];
        float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it.out) +
                                            (int64_t)(head0 + h) * it.o_s1);
        *reinterpret_cast<float4*>(o + 4 * lane) =
            make_float4(acc[h][0] * inv, acc[h][1] * inv, acc[h][2] * inv, acc[h][3] * inv);
      }
    }
    return;
  }
  float* rec = p.part + (int64_t)wid * REC;
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
}

template <int D, typename KT, int G>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(2)))
void decode_kernel(const DecodeParams p) {
  decode_body<D, KT, G, 1>(p);
}

template <int D, typename KT, int G>
__global__ __launch_bounds__(kWave) void decode_kernel_deep(const DecodeParams p) {
  decode_body<D, KT, G, 2>(p);
}

// Combines the nw run records of one (group, head) per workgroup. Thread t
// owns output dims 4 (t % (D/4)) .. +3 and the records s = t / (D/4) + k*RS:
// it keeps a running (m, l, acc) over its few records (all loads independent,
// so one memory round trip), then the RS partials of each dim combine through
// LDS with the same stable rescaling.
template <int D, int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(const DecodeParams p) {
  constexpr int HDR = record_header(G);
  constexpr int REC = HDR + G * D;
  constexpr int C4 = D / 4;          // threads per record (one float4 of dims each)
  constexpr int RS = 256 / C4;       // record subsets
  __shared__ float sm[RS], sl[RS];
  __shared__ float4 sa[RS][C4];
  const int per_item = p.n_head_kv * p.n_chunks;
  const int grp = blockIdx.x / G;
  const int h = blockIdx.x % G;
  const DecodeItem& it = p.item[grp / per_item];
  const int S = it.nw;
  if (S == 1) return;  // written by its only run
  const int gl = grp % per_item;
  const int g = gl / p.n_chunks;
  const int hc = gl % p.n_chunks;
  const int head = g * p.n_rep + hc * G + h;
  const float* base = p.part + (int64_t)(it.wave0 + gl * S) * REC;
  const int c4 = threadIdx.x % C4, sub = threadIdx.x / C4;

  float m = -INFINITY, l = 0.f;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
  for (int s = sub; s < S; s += RS) {
    const float* r = base + (int64_t)s * REC;
    const float ms = r[h], ls = r[G + h];
    const float4 as = *reinterpret_cast<const float4*>(r + HDR + h * D + 4 * c4);
    const float mn = fmaxf(m, ms);
    const float wo = fast_exp2(m - mn), wn = fast_exp2(ms - mn);
    l = l * wo + ls * wn;
    a.x = a.x * wo + as.x * wn;
    a.y = a.y * wo + as.y * wn;
    a.z = a.z * wo + as.z * wn;
    a.w = a.w * wo + as.w * wn;
    m = mn;
  }
  if (c4 == 0) {
    sm[sub] = m;
    sl[sub] = l;
  }
  sa[sub][c4] = a;
  __syncthreads();
  if (sub != 0) return;
  float mx = -INFINITY;
  for (int k = 0; k < RS; ++k) mx = fmaxf(mx, sm[k]);
  float lt = 0.f;
  float4 at = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k = 0; k < RS; ++k) {
    const float wk = sm[k] == -INFINITY ? 0.f : fast_exp2(sm[k] - mx);  // subset with no record
    lt += wk * sl[k];
    const float4 ak = sa[k][c4];
    at.x += wk * ak.x;
    at.y += wk * ak.y;
    at.z += wk * ak.z;
    at.w += wk * ak.w;
  }
  const float inv = 1.f / lt;
  float* o = reinterpret_cast<float*>(reinterpret_cast<char*>(it.out) + (int64_t)head * it.o_s1);
  *reinterpret_cast<float4*>(o + 4 * c4) = make_float4(at.x * inv, at.y * inv, at.z * inv, at.w * inv);
}

// Depth 1 (two waves per SIMD) for head_dim 64; head_dim 128 tiles do not fit
// 256 registers with a refill in flight, so they run at depth 2 (one wave per
// SIMD). MI_HIP_DECODE_DEPTH=1|2 overrides (tuning).
int decode_depth(int head_dim) {
  static const int forced = [] {
    const char* e = std::getenv("MI_HIP_DECODE_DEPTH");
    return e && (e[0] == '1' || e[0] == '2') ? e[0] - '0' : 0;
  }();
  return forced ? forced : (head_dim == 64 ? 1 : 2);
}

template <int D, typename KT, int G>
static hipError_t launch_decode_t(const DecodeParams& p, int max_nw, hipStream_t stream) {
  if (decode_depth(D) == 2)
    hipLaunchKernelGGL((decode_kernel_deep<D, KT, G>), dim3((unsigned)p.n_waves), dim3(kWave), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((decode_kernel<D, KT, G>), dim3((unsigned)p.n_waves), dim3(kWave), 0,
                       stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_nw <= 1) return e;
  const unsigned groups = (unsigned)(p.n_items * p.n_head_kv * p.n_chunks);
  hipLaunchKernelGGL((decode_merge_kernel<D, G>), dim3(groups * G), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <int D, typename KT>
static hipError_t launch_decode_g(const DecodeParams& p, int g, int max_nw, hipStream_t stream) {
  switch (g) {
    case 1: return launch_decode_t<D, KT, 1>(p, max_nw, stream);
    case 2: return launch_decode_t<D, KT, 2>(p, max_nw, stream);
    case 4: return launch_decode_t<D, KT, 4>(p, max_nw, stream);
    case 7: return launch_decode_t<D, KT, 7>(p, max_nw, stream);
    case 8: return launch_decode_t<D, KT, 8>(p, max_nw, stream);
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
  return (size_t)record_header(group) + (size_t)group * head_dim;
}

hipError_t launch_decode(const DecodeParams& p, int head_dim, bool f16, int group, int max_nw,
                         hipStream_t stream) {
  if (head_dim == 64)
    return f16 ? launch_decode_g<64, _Float16>(p, group, max_nw, stream)
               : launch_decode_g<64, float>(p, group, max_nw, stream);
  if (head_dim == 128)
    return f16 ? launch_decode_g<128, _Float16>(p, group, max_nw, stream)
               : launch_decode_g<128, float>(p, group, max_nw, stream);
  return hipErrorInvalidValue;
}

}  // namespace mi
