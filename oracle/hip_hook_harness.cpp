// hip_hook_harness.cpp -- TEST INFRASTRUCTURE (never product code): drives
// the product's executor hook from the reference engine's own executor.
//
// Linked into the reference CLI (src/main.cpp and the core sources, compiled
// where they lie) with GNU ld's --wrap, so that the reference's unmodified
// call sites reach the product library through the four integration points
// a maintainer adds to the engine:
//   mi_compute_forward      (src/ops_cpu.cpp:481; called by every pool thread,
//                            src/threadpool.cpp:171-180, by the pool-less
//                            src/graph.cpp:75-83, and by the dump path,
//                            src/model_qwen2.cpp:647-672)
//                           -> mi_hip_compute_forward first; the CPU kernel
//                              only when the hook declines the node
//   mi_gallocr_alloc_graph  (src/gallocr.cpp; called once per forward step,
//                            src/model_qwen2.cpp:630, before either path)
//                           -> then mi_hip_graph_prepare on the step's graph
//   mi_kv_cache_init / _free (src/model_qwen2.cpp:557-605)
//                           -> a device cache of the same shape, each layer's
//                              host K/V tensor bound to it; for a head_dim the
//                              fused kernels do not take, no device cache: the
//                              attention nodes then run on the node kernels
//                              (mi_hip_set_host_nodes)
// The wrapped symbols are the reference's C++ names, so the wrappers carry
// their mangled names (the Makefile lists the same names to --wrap).
//
// At exit it reports, on stderr, the device allocations made after the last
// KV cache was created ("mi_hip_hook: device allocations after init N") and
// how many nodes the hook ran ("nodes on device M").
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>

#include "gallocr.h"
#include "graph.h"
#include "model_qwen2.h"
#include "ops_cpu.h"
// The reference's tensor.h and graph.h above declare the node layout that
// include/mi_tensor.h restates (layout-identical; tests/test_abi.py checks
// sizeof/offsetof): keep the reference's and take only the API declarations.
#define MI_TENSOR_H
#include "mi_hip_attn.h"

namespace {

std::mutex g_mu;
std::map<const mi_kv_cache*, mi_hip_kv*> g_caches;
uint64_t g_mallocs_at_init = 0;
std::atomic<long> g_device_nodes{0};
std::atomic<bool> g_reported{false};

void die(const char* what) {
  std::fprintf(stderr, "mi_hip_hook: %s: %s\n", what, mi_hip_last_error());
  std::abort();
}

void report() {
  if (g_reported.exchange(true)) return;
  mi_hip_alloc_stats st{};
  if (mi_hip_get_alloc_stats(&st) == MI_HIP_OK)
    std::fprintf(stderr, "mi_hip_hook: device allocations after init %llu, nodes on device %ld\n",
                 (unsigned long long)(st.n_malloc - g_mallocs_at_init), g_device_nodes.load());
}

}  // namespace

extern "C" {

void __real__Z18mi_compute_forwardP9mi_tensorii(mi_tensor* dst, int ith, int nth);
void __wrap__Z18mi_compute_forwardP9mi_tensorii(mi_tensor* dst, int ith, int nth) {
  const int rc = mi_hip_compute_forward(dst, ith, nth);
  if (rc > 0) {
    if (ith == 0) g_device_nodes++;
    return;
  }
  if (rc < 0) die("mi_hip_compute_forward");
  __real__Z18mi_compute_forwardP9mi_tensorii(dst, ith, nth);
}

void __real__Z22mi_gallocr_alloc_graphP10mi_gallocrP9mi_cgraph(mi_gallocr* galloc, mi_cgraph* g);
void __wrap__Z22mi_gallocr_alloc_graphP10mi_gallocrP9mi_cgraph(mi_gallocr* galloc, mi_cgraph* g) {
  __real__Z22mi_gallocr_alloc_graphP10mi_gallocrP9mi_cgraph(galloc, g);
  if (mi_hip_graph_prepare(g) != MI_HIP_OK) die("mi_hip_graph_prepare");
}

mi_kv_cache* __real__Z16mi_kv_cache_initRK16mi_qwen2_hparamsRK16mi_qwen2_weightsiRK20mi_threadpool_params(
    const mi_qwen2_hparams& hp, const mi_qwen2_weights& w, int n_ctx, const mi_threadpool_params& tp);
mi_kv_cache* __wrap__Z16mi_kv_cache_initRK16mi_qwen2_hparamsRK16mi_qwen2_weightsiRK20mi_threadpool_params(
    const mi_qwen2_hparams& hp, const mi_qwen2_weights& w, int n_ctx, const mi_threadpool_params& tp) {
  mi_kv_cache* kv =
      __real__Z16mi_kv_cache_initRK16mi_qwen2_hparamsRK16mi_qwen2_weightsiRK20mi_threadpool_params(hp, w, n_ctx, tp);
  if (!kv) return kv;
  if (mi_hip_init(0) != MI_HIP_OK) die("mi_hip_init");
  if (mi_hip_set_host_nodes(1) != MI_HIP_OK) die("mi_hip_set_host_nodes");
  static std::once_flag once;
  std::call_once(once, [] { std::atexit(report); });  // if the cache is never freed
  mi_hip_kv_desc d{hp.n_layer, n_ctx, hp.n_head_kv, hp.head_dim, hp.n_head, 0 /* F32 */};
  mi_hip_kv* hk = nullptr;
  const int crc = mi_hip_kv_create(&d, &hk);
  if (crc == MI_HIP_E_UNSUPPORTED) {  // host cache; attention on the node kernels
    std::fprintf(stderr, "mi_hip_hook: no device cache (%s)\n", mi_hip_last_error());
    std::lock_guard<std::mutex> lk(g_mu);
    mi_hip_alloc_stats st{};
    if (mi_hip_get_alloc_stats(&st) == MI_HIP_OK) g_mallocs_at_init = st.n_malloc;
    return kv;
  }
  if (crc != MI_HIP_OK) die("mi_hip_kv_create");
  for (int l = 0; l < hp.n_layer; l++) {
    if (mi_hip_kv_bind(hk, l, 0, kv->k[l]) != MI_HIP_OK) die("mi_hip_kv_bind K");
    if (mi_hip_kv_bind(hk, l, 1, kv->v[l]) != MI_HIP_OK) die("mi_hip_kv_bind V");
  }
  std::lock_guard<std::mutex> lk(g_mu);
  g_caches[kv] = hk;
  mi_hip_alloc_stats st{};
  if (mi_hip_get_alloc_stats(&st) == MI_HIP_OK) g_mallocs_at_init = st.n_malloc;
  return kv;
}

void __real__Z16mi_kv_cache_freeP11mi_kv_cache(mi_kv_cache* kv);
void __wrap__Z16mi_kv_cache_freeP11mi_kv_cache(mi_kv_cache* kv) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_caches.find(kv);
    if (it != g_caches.end()) {
      report();
      mi_hip_kv_destroy(it->second);
      g_caches.erase(it);
    }
  }
  __real__Z16mi_kv_cache_freeP11mi_kv_cache(kv);
}

}  // extern "C"
