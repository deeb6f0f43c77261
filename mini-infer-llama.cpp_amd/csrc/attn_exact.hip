// attn_exact.hip -- ATTN_QK -> causal SOFTMAX -> ATTN_KQV in the reference's
// own operation order (src/ops_cpu.cpp:304-410), bit for bit:
//
//   S_i  = sum_d K[d, kvh, i] * Q[d, h, j]     d ascending, product and sum
//                                              each rounded (no fused multiply-add)
//   v_i  = S_i * scale;  m = max_i v_i         i < a = min(n_past + j + 1, n_kv)
//   e_i  = expf(v_i - m)                       the host C library's expf (libm_ref.h)
//   sum  = sum_i e_i                           i ascending
//   P_i  = e_i * (1 / sum)
//   O[o] = sum_t V[o, kvh, t] * P_t            t ascending (masked t add +-0, skipped)
//
// Rows whose keys' V fit in LDS (a * head_dim * 4 <= kExactStageBytes) run
// attn_exact_staged_kernel: 256 threads per (token j, head h); the row's K
// rows come into LDS (LDS-direct, coalesced) and the threads form one key's
// score each from there; then three waves bring the V rows over the K rows
// while wave 0 forms the maximum, the exponentials and (lane 0) the ordered
// sum; then each output element's lane runs its ordered V sum from LDS.
// Longer rows run attn_exact_kernel: one wave
// per (token, head), lanes splitting the keys and then the output elements,
// V read from global memory. Either way the ordered sums make a row's cost
// linear in its key count on one lane: this is the checking path for
// whole-model parity (token ids equal to the reference engine's), not the
// throughput path (decode.hip / prefill.hip).
#include <cmath>

#include "attn_common.h"
#include "kernels.h"

#define MI_LIBM_HD __host__ __device__
#include "libm_ref.h"

namespace mi {

static __constant__ uint64_t kExpfTab[32] = MI_EXPF_TABLE;

__global__ __launch_bounds__(kWave) void attn_exact_kernel(const ExactAttn p) {
#pragma clang fp contract(off)
  extern __shared__ float prob[];
  __shared__ float s_inv;
  const int lane = threadIdx.x;
  const int h = blockIdx.x % p.n_head;
  const int j = blockIdx.x / p.n_head;
  const int kvh = h / p.n_rep;
  const int D = p.head_dim;
  const int a = min(p.n_past + j + 1, p.n_past + p.n_tokens);
  const float* q = reinterpret_cast<const float*>(p.q + h * p.q_s1 + (int64_t)j * p.q_s2);
  float mx = -INFINITY;
  for (int i = lane; i < a; i += kWave) {
    const float* kr = reinterpret_cast<const float*>(p.k + kvh * p.k_s1 + (int64_t)i * p.k_s2);
    float acc = 0.0f;
#pragma unroll 16  // (the row's loads in flight together)
    for (int d = 0; d < D; d += 4) {
      const float4 kv = *reinterpret_cast<const float4*>(kr + d);
      const float4 qv = *reinterpret_cast<const float4*>(q + d);
      acc = acc + kv.x * qv.x;
      acc = acc + kv.y * qv.y;
      acc = acc + kv.z * qv.z;
      acc = acc + kv.w * qv.w;
    }
    const float v = acc * p.scale;
    prob[i] = v;
    mx = v > mx ? v : mx;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off);
    mx = o > mx ? o : mx;
  }
  for (int i = lane; i < a; i += kWave) prob[i] = expf_ref(prob[i] - mx, kExpfTab);
  __syncthreads();
  if (lane == 0) {
    float sum = 0.0f;
    for (int i = 0; i < a; ++i) sum = sum + prob[i];
    s_inv = (float)(1.0 / (double)sum);  // the correctly rounded 1.0f / sum
  }
  __syncthreads();
  const float inv = s_inv;
  for (int i = lane; i < a; i += kWave) prob[i] = prob[i] * inv;
  __syncthreads();
  float* out = reinterpret_cast<float*>(p.out + h * p.o_s1 + (int64_t)j * p.o_s2);
  const char* vbase = p.v + kvh * p.v_s1;
  for (int o = lane; o < D; o += kWave) {
    float acc = 0.0f;
#pragma unroll 16  // (16 keys' loads in flight ahead of the ordered additions)
    for (int t = 0; t < a; ++t)
      acc = acc + *reinterpret_cast<const float*>(vbase + (int64_t)t * p.v_s2 + 4 * o) * prob[t];
    out[o] = acc;
  }
}

constexpr int kExactStageBytes = 128 * 1024;  // the staged kernel's V rows
constexpr int kExactThreads = 256;

// LDS of the staged kernel for rows of up to n_kv keys: the V rows (whole 1 KB
// transfers), the probabilities, expf's table, the wave maxima and 1 / sum.
// The V rows and the probabilities have 16 entries of room past n_kv: the
// ordered sums read each chunk of 16 ahead of its additions, the one past
// the last whole chunk too (read, never added).
__host__ __device__ inline int exact_staged_vbytes(int n_kv, int d) {
  return ((n_kv + 16) * d * 4 + 1023) & ~1023;
}
__host__ __device__ inline int exact_staged_lds(int n_kv, int d) {
  return exact_staged_vbytes(n_kv, d) + 4 * (n_kv + 16) + 32 * 8 + 4 * 4 + 16;
}

// The ordered sums of the staged kernel, in chunks of 16 terms: chunk c + 1
// is read from LDS before chunk c's additions, so that the chain of additions
// does not wait for each read. Terms past the last whole chunk go one by one.
// s + p[0] + p[1] + ... + p[n - 1] (p 16-byte aligned, 16 floats readable past n)
__device__ __forceinline__ float exact_sum(const float* p, int n) {
#pragma clang fp contract(off)
  const float4* p4 = reinterpret_cast<const float4*>(p);
  float s = 0.0f;
  float4 x[4], y[4];
  auto get = [&](float4 (&b)[4], int c) {
#pragma unroll
    for (int u = 0; u < 4; ++u) b[u] = p4[4 * c + u];
  };
  auto add = [&](const float4 (&b)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      s = s + b[u].x;
      s = s + b[u].y;
      s = s + b[u].z;
      s = s + b[u].w;
    }
  };
  const int nch = n >> 4;
  get(x, 0);
  int c = 0;
  // (the scheduler would otherwise sink each chunk's reads below the
  // additions before them)
  for (; c + 1 < nch; c += 2) {
    get(y, c + 1);
    __builtin_amdgcn_sched_barrier(0);
    add(x);
    get(x, c + 2);
    __builtin_amdgcn_sched_barrier(0);
    add(y);
  }
  if (c < nch) add(x);
  for (int i = 16 * nch; i < n; ++i) s = s + p[i];
  return s;
}

// acc + v[0] * p[0] + v[D] * p[1] + ... + v[(n - 1) D] * p[n - 1], each
// product and sum rounded (v: one output element's column of V rows D floats
// apart; 16 rows and probabilities readable past n). The products do not
// depend on the running sum: chunk c + 1's 16 are formed between chunk c's
// additions, so each addition waits only for the one before it, not for a
// multiplication issued just before it. (The same products, added in the
// same order: the same bits.)
template <int D>
__device__ __forceinline__ float exact_dot(const float* v, const float* p, int n) {
#pragma clang fp contract(off)
  const float4* p4 = reinterpret_cast<const float4*>(p);
  float acc = 0.0f;
  float va[16], vb[16];
  float4 pa[4], pb[4];
  float ra[16], rb[16];  // products
  auto get = [&](float (&vv)[16], float4 (&pp)[4], int c) {
#pragma unroll
    for (int u = 0; u < 16; ++u) vv[u] = v[(16 * c + u) * D];
#pragma unroll
    for (int u = 0; u < 4; ++u) pp[u] = p4[4 * c + u];
  };
  auto prod = [&](float (&r)[16], const float (&vv)[16], const float4 (&pp)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      r[4 * u] = vv[4 * u] * pp[u].x;
      r[4 * u + 1] = vv[4 * u + 1] * pp[u].y;
      r[4 * u + 2] = vv[4 * u + 2] * pp[u].z;
      r[4 * u + 3] = vv[4 * u + 3] * pp[u].w;
    }
  };
  // chunk r's additions, chunk (vv, pp)'s products into rn between them
  auto add_prod = [&](const float (&r)[16], float (&rn)[16], const float (&vv)[16], const float4 (&pp)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc = acc + r[4 * u];
      rn[4 * u] = vv[4 * u] * pp[u].x;
      acc = acc + r[4 * u + 1];
      rn[4 * u + 1] = vv[4 * u + 1] * pp[u].y;
      acc = acc + r[4 * u + 2];
      rn[4 * u + 2] = vv[4 * u + 2] * pp[u].z;
      acc = acc + r[4 * u + 3];
      rn[4 * u + 3] = vv[4 * u + 3] * pp[u].w;
    }
  };
  auto add = [&](const float (&r)[16]) {
#pragma unroll
    for (int t = 0; t < 16; ++t) acc = acc + r[t];
  };
  const int nch = n >> 4;
  if (nch > 0) {
    get(va, pa, 0);
    prod(ra, va, pa);
    if (nch > 1) get(vb, pb, 1);
    int c = 0;
    // ra: chunk c's products; vb, pb: chunk c + 1's values
    for (; c + 2 < nch; c += 2) {
      get(va, pa, c + 2);
      __builtin_amdgcn_sched_barrier(0);
      add_prod(ra, rb, vb, pb);
      get(vb, pb, c + 3);  // (c + 3 <= nch: at most the chunk past the last whole one)
      __builtin_amdgcn_sched_barrier(0);
      add_prod(rb, ra, va, pa);
    }
    if (c + 1 < nch) {
      add_prod(ra, rb, vb, pb);
      add(rb);
    } else {
      add(ra);
    }
  }
  for (int t = 16 * nch; t < n; ++t) acc = acc + v[t * D] * p[t];
  return acc;
}

// D: head_dim (64 or 128). The row's K rows come into LDS first, into the
// region that later holds its V rows: LDS-direct requests of whole 1 KB
// (where a thread loading its own key row touches one cache line per lane
// and instruction), 16-byte slots XOR-swizzled by row so that one row per
// lane reads free of bank conflicts. After the scores, waves 1-3 bring the V
// rows over the K rows while wave 0 forms the maximum, the exponentials and
// the ordered sum; the barriers do not wait for vector memory (wg_barrier),
// each wave waits for its own requests.
template <int D>
__global__ __launch_bounds__(kExactThreads) void attn_exact_staged_kernel(const ExactAttn p) {
#pragma clang fp contract(off)
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  extern __shared__ __attribute__((aligned(16))) char ex_lds[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int h = blockIdx.x % p.n_head;
  const int j = blockIdx.x / p.n_head;
  const int kvh = h / p.n_rep;
  const int a = min(p.n_past + j + 1, p.n_past + p.n_tokens);
  const int n_kv = p.n_past + p.n_tokens;
  const int vbytes = exact_staged_vbytes(n_kv, D);
  constexpr int PPR = D / 4;  // 16-byte pieces per row
  float* const vl = reinterpret_cast<float*>(ex_lds);  // K, later V, row t at vl + t D
  float* const prob = reinterpret_cast<float*>(ex_lds + vbytes);
  uint64_t* const tab = reinterpret_cast<uint64_t*>(ex_lds + vbytes + 4 * n_kv);
  float* const red = reinterpret_cast<float*>(tab + 32);
  const uint64_t te = kExpfTab[lane & 31];  // requested first: loads complete in order
  const int pieces = a * PPR;
  // rows of one KV head from base into LDS: piece i is physical slot i % PPR
  // of row i / PPR, which holds logical slot (i % PPR) ^ sw(row); pieces past
  // the row arrive as zeros. Waves w0.. w0 + nw - 1 share the requests.
  auto rows_to_lds = [&](const char* base, int64_t s2, bool swizzle, int w0, int nw) __attribute__((always_inline)) {
    const unsigned size = (unsigned)((int64_t)(a - 1) * s2 + 4 * D);
    const rsrc_t r = make_rsrc(base, size);
    for (int i0 = kWave * (wv - w0); i0 < pieces; i0 += kWave * nw) {
      const int i = i0 + lane, row = i / PPR, slot = i % PPR;
      const int ls = swizzle ? slot ^ swz<PPR>(row) : slot;
      const unsigned off = i < pieces ? (unsigned)((int64_t)row * s2 + 16 * ls) : size;
      dma16(r, (lds_t*)ex_lds + 16 * i0, off);
    }
  };
  rows_to_lds(p.k + kvh * p.k_s1, p.k_s2, true, 0, kExactThreads / kWave);
  // this wave's query elements into registers meanwhile
  const float* q = reinterpret_cast<const float*>(p.q + h * p.q_s1 + (int64_t)j * p.q_s2);
  float4 qv[PPR];
#pragma unroll
  for (int u = 0; u < PPR; ++u) qv[u] = *reinterpret_cast<const float4*>(q + 4 * u);
  wait_vmem<0>();  // this wave's K requests (and the query) have landed
  wg_barrier();
  // one key's score per thread, d ascending, product and sum each rounded
  float mx = -INFINITY;
  for (int i = tid; i < a; i += kExactThreads) {
    const lds_t* const rowp = (const lds_t*)ex_lds + i * (4 * D);
    // the D products first (independent), then their sum in order
    float pr[D];
#pragma unroll
    for (int u = 0; u < PPR; ++u) {
      const f32x4_t kv = lds_load<f32x4_t>(rowp + 16 * (u ^ swz<PPR>(i)));
      pr[4 * u] = kv.x * qv[u].x;
      pr[4 * u + 1] = kv.y * qv[u].y;
      pr[4 * u + 2] = kv.z * qv[u].z;
      pr[4 * u + 3] = kv.w * qv[u].w;
    }
    float acc = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) acc = acc + pr[d];
    const float v = acc * p.scale;
    prob[i] = v;
    mx = v > mx ? v : mx;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off);
    mx = o > mx ? o : mx;
  }
  if (tid < 32) tab[tid] = te;
  if (lane == 0) red[wv] = mx;
  wg_barrier();  // the scores are in LDS and every K row has been read
  if (wv > 0) {
    rows_to_lds(p.v + kvh * p.v_s1, p.v_s2, false, 1, kExactThreads / kWave - 1);
    wait_vmem<0>();  // this wave's V requests have landed
  } else {
    mx = red[0];
    for (int w = 1; w < kExactThreads / kWave; ++w) mx = red[w] > mx ? red[w] : mx;
    for (int i = lane; i < a; i += kWave) prob[i] = expf_ref(prob[i] - mx, tab);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's exponentials are in LDS
    if (lane == 0) {
      const float sum = exact_sum(prob, a);
      red[4] = (float)(1.0 / (double)sum);  // the correctly rounded 1.0f / sum
    }
  }
  wg_barrier();  // the V rows and 1 / sum
  const float inv = red[4];
  for (int i = tid; i < a; i += kExactThreads) prob[i] = prob[i] * inv;
  wg_barrier();
  if (tid < D) {
    const float acc = exact_dot<D>(vl + tid, prob, a);
    float* out = reinterpret_cast<float*>(p.out + h * p.o_s1 + (int64_t)j * p.o_s2);
    out[tid] = acc;
  }
}

hipError_t launch_attn_exact(const ExactAttn& p, hipStream_t stream) {
  const int n_kv = p.n_past + p.n_tokens;
  if ((int64_t)n_kv * p.head_dim * 4 <= kExactStageBytes && (p.head_dim == 64 || p.head_dim == 128) &&
      p.v_s2 % 4 == 0 && reinterpret_cast<uintptr_t>(p.v) % 4 == 0 && p.v_s1 % 4 == 0) {
    static const hipError_t attr = [] {
      hipError_t e = hipFuncSetAttribute((const void*)&attn_exact_staged_kernel<64>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         exact_staged_lds(kExactStageBytes / (4 * 64), 64));
      if (e == hipSuccess)
        e = hipFuncSetAttribute((const void*)&attn_exact_staged_kernel<128>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                exact_staged_lds(kExactStageBytes / (4 * 128), 128));
      return e;
    }();
    if (attr != hipSuccess) return attr;
    const dim3 grid((unsigned)(p.n_tokens * p.n_head));
    const size_t lds = (size_t)exact_staged_lds(n_kv, p.head_dim);
    if (p.head_dim == 64)
      hipLaunchKernelGGL(attn_exact_staged_kernel<64>, grid, dim3(kExactThreads), lds, stream, p);
    else
      hipLaunchKernelGGL(attn_exact_staged_kernel<128>, grid, dim3(kExactThreads), lds, stream, p);
    return hipGetLastError();
  }
  const size_t lds = (size_t)n_kv * sizeof(float);
  static const hipError_t attr = hipFuncSetAttribute(
      (const void*)&attn_exact_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kExactMaxKeys * 4);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(attn_exact_kernel, dim3((unsigned)(p.n_tokens * p.n_head)), dim3(kWave), lds,
                     stream, p);
  return hipGetLastError();
}

}  // namespace mi
