// memread.hip -- the measured read-bandwidth ceiling of the device: a
// read-and-accumulate pass over a buffer, as tools/bench_memread.cpp measures
// the host's (a sequential load-and-add over at least 1 GiB, one reduced sum
// per worker, no writes to the source). The accumulation keeps every loaded
// value live, so no load can be dropped.
//
// Workgroup w (512 threads) owns the 16-byte pieces [w * per_wg, (w + 1) *
// per_wg) of the buffer; each thread keeps 8 loads of 16 bytes in flight
// (consecutive threads read consecutive pieces, so every load instruction of
// a wave covers 1 KB of contiguous memory) and the workgroup writes one float.
// The loads are nontemporal, as the decode kernels' cache streams are: data
// read once does not displace what the caches hold (on the 100.7 MB cache
// read of 24 layers x n_kv 4096 this is worth about 2 us of 18).
#include "kernels.h"
#include "mi_hip_attn.h"

namespace mi {

constexpr int kMemreadThreads = 512;
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kMemreadUnroll = 8;

__global__ __launch_bounds__(kMemreadThreads) void memread_kernel(const f32x4_t* src, int64_t n4,
                                                                 int64_t per_wg, float* sums) {
  const int64_t b0 = (int64_t)blockIdx.x * per_wg;
  const int64_t b1 = min(b0 + per_wg, n4);
  constexpr int64_t step = kMemreadThreads;
  f32x4_t acc[kMemreadUnroll];
#pragma unroll
  for (int u = 0; u < kMemreadUnroll; ++u) acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  int64_t i = b0 + threadIdx.x;
  // every piece read here is below b1 <= n4
  for (; i + (kMemreadUnroll - 1) * step < b1; i += kMemreadUnroll * step) {
    f32x4_t v[kMemreadUnroll];
#pragma unroll
    for (int u = 0; u < kMemreadUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * step);
#pragma unroll
    for (int u = 0; u < kMemreadUnroll; ++u) acc[u] += v[u];
  }
  for (; i < b1; i += step) acc[0] += __builtin_nontemporal_load(src + i);
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < kMemreadUnroll; ++u) s += (acc[u].x + acc[u].y) + (acc[u].z + acc[u].w);
  for (int off = kWave / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
  __shared__ float part[kMemreadThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int w = 0; w < kMemreadThreads / kWave; ++w) t += part[w];
    sums[blockIdx.x] = t;
  }
}

hipError_t launch_memread(const void* src, size_t bytes, float* sums, int n_sums, hipStream_t stream) {
  const int64_t n4 = (int64_t)(bytes / 16);
  const int64_t per_wg = (n4 + n_sums - 1) / n_sums;
  hipLaunchKernelGGL(memread_kernel, dim3((unsigned)n_sums), dim3(kMemreadThreads), 0, stream,
                     static_cast<const f32x4_t*>(src), n4, per_wg, sums);
  return hipGetLastError();
}

}  // namespace mi

extern "C" int mi_hip_memread(const void* src, size_t bytes, float* sums, int32_t n_sums, void* stream) {
  using namespace mi;
  if (!src || !sums) return rt_fail(MI_HIP_E_INVALID, "memread: src or sums is NULL");
  if (bytes == 0 || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return rt_fail(MI_HIP_E_INVALID, "memread: bytes must be a nonzero multiple of 16 and src 16-byte aligned");
  if (n_sums < 1 || n_sums > 65536) return rt_fail(MI_HIP_E_INVALID, "memread: n_sums out of [1, 65536]");
  if (const int rc = rt_bind()) return rc;
  const hipError_t e = launch_memread(src, bytes, sums, n_sums, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MI_HIP_OK : rt_hip_fail(e, "memread launch");
}
