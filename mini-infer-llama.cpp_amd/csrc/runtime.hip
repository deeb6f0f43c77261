// runtime.hip -- host side of the C ABI declared in include/mi_hip_attn.h.
//
// Responsibilities: argument validation (every entry point returns a status
// and never throws), device-allocation accounting, the device-resident KV
// cache, launch planning for the decode and prefill kernels, the node-level
// operators on device tensors, and the executor hook that lets the engine's
// host graph route its attention nodes here.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <unordered_map>

#include "attn_common.h"
#include "kernels.h"
#include "mi_hip_attn.h"

namespace {

// ---------------------------------------------------------------------------
// Errors
// ---------------------------------------------------------------------------
thread_local char t_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(t_err, sizeof t_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(e == hipErrorOutOfMemory ? MI_HIP_E_NOMEM : MI_HIP_E_RUNTIME, "%s: %s", what,
              hipGetErrorString(e));
}

#define MI_TRY_HIP(expr, what)            \
  do {                                    \
    hipError_t e_ = (expr);               \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

// ---------------------------------------------------------------------------
// Library state and device allocation accounting
// ---------------------------------------------------------------------------
// Tuning knobs, read from the environment once, at mi_hip_init:
//   MI_HIP_DECODE_KPG=n    forces n workgroups per decode group
//   MI_HIP_DECODE_EARLY=0  disables the early merge protocol
//   MI_HIP_DECODE_SOLO=n   groups of at most n ring loads' worth of sub-tiles
//                          get one workgroup (no cross-workgroup merge)
//   MI_HIP_DECODE_CLAIM=n  claim sub-tiles from device counters when each wave
//                          streams at least n ring loads (0, the default: never;
//                          measured slower on MI355X at every shape tried, since a
//                          claim's round trip holds up the loads issued after it)
//   MI_HIP_DECODE_HSPLIT=0 keeps a group's heads together in every launch; 1 cuts
//                          them only when every group of a launch has one
//                          workgroup; 2 (the default) also in launches whose
//                          groups merge parts (see plan_decode)
struct Knobs {
  int stream_min = 0;  // AUTO: streaming kernel from this many sub-tiles per wave (0: never)
  int kpg = 0;
  int early = 1;
  int solo = 1;
  int claim = 0;
  int hsplit = 2;
};

struct State {
  std::mutex mu;
  int device = -1;
  bool ready = false;
  std::atomic<uint64_t> n_malloc{0}, n_free{0}, live{0}, peak{0};
  std::atomic<uint64_t> limit{0};
  int n_cu = 0;  // compute units of the device
  Knobs knobs;
  std::atomic<int> deterministic{1};  // fixed per-wave takes in the fused kernels
  std::atomic<int> prefill_mode{MI_HIP_PREFILL_AUTO};  // matrix cores of the prefill kernel
  std::atomic<int> decode_mode{MI_HIP_DECODE_AUTO};          // matrix cores of the decode kernel
  mi_hip_workspace* default_ws = nullptr;  // for calls that name no workspace
  mi_hip_workspace* scratch_ws = nullptr;  // this device's entry of scratch_by_device
  // Host-resident attention nodes run on the node kernels (opt-in): a staging
  // buffer that grows to the largest node seen, and a stream for it.
  std::atomic<int> host_nodes{0};
  std::mutex node_mu;
  char* node_stage = nullptr;
  size_t node_stage_bytes = 0;
  hipStream_t node_stream = nullptr;
};
State g;

// The no-allocation entry point's workspace of each device, kept for the
// life of the process like the array it lies over: its launch stamp and
// counter-set state must continue across mi_hip_shutdown / mi_hip_init,
// because the array keeps the records and counters of every earlier call.
constexpr int kMaxDevices = 64;
mi_hip_workspace* scratch_by_device[kMaxDevices] = {};

int dev_alloc(void** p, size_t bytes, const char* what) {
  const uint64_t lim = g.limit.load();
  if (lim && g.live.load() + bytes > lim)
    return fail(MI_HIP_E_NOMEM, "%s: %zu bytes would exceed the allocation limit of %llu", what,
                bytes, (unsigned long long)lim);
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return hip_fail(e, what);
  g.n_malloc++;
  const uint64_t now = g.live.fetch_add(bytes) + bytes;
  uint64_t pk = g.peak.load();
  while (now > pk && !g.peak.compare_exchange_weak(pk, now)) {
  }
  return MI_HIP_OK;
}

void dev_free(void* p, size_t bytes) {
  if (!p) return;
  (void)hipFree(p);
  g.n_free++;
  g.live.fetch_sub(bytes);
}

int bind_device() {
  if (!g.ready) return fail(MI_HIP_E_STATE, "mi_hip_init has not been called");
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != g.device) MI_TRY_HIP(hipSetDevice(g.device), "hipSetDevice");
  return MI_HIP_OK;
}

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return v && *v ? std::atoi(v) : dflt;
}

// ---------------------------------------------------------------------------
// Launch planning
// ---------------------------------------------------------------------------
constexpr float kLog2e = 1.4426950408889634f;

// Decode launch plan. Every group (item, KV head, head chunk) gets kpg
// workgroups, in proportion to its share of the launch's sub-tiles so that the
// launch has about one workgroup per CU; at least one, and no more than leave
// each wave one sub-tile. A group of at most knobs.solo rounds gets one
// workgroup: its loads are one latency anyway, and a cross-workgroup merge
// would cost more than it saves. When a group is
// long enough that each of its waves streams at least knobs.claim ring loads,
// sub-tiles are claimed dynamically (so that a claim's round trip hides behind
// a ring cycle); otherwise each workgroup owns every kpg-th sub-tile of its
// group.
//
// Head split: when every group of a launch gets one workgroup, the launch is
// bound by each workgroup's arithmetic over its heads (its loads are one
// latency), not by the memory system; a group of more than 4 heads is then
// cut into two chunks of ceil(G / 2) and G - ceil(G / 2) heads, each with a
// workgroup of its own. Both read the group's K/V rows (twice the requests,
// served from L2 for the second), each does half the arithmetic, and no merge
// is needed since each chunk owns its heads' outputs. The same holds for
// launches whose groups merge parts, as long as the split keeps every group's
// part count (so its workgroups double and no part streams more than before)
// and the launch within one workgroup per CU: each part then streams its
// positions for half the heads, and each chunk's parts merge among themselves
// (one layer of the 0.5B shape from HBM, n_kv 257..1024: 7.2-8.0 -> 6.6-7.0 us
// per launch, 2048: 7.8 -> 7.1, 4096: 8.05 -> 7.5; at n_kv 8192, where the
// split halves the part count, 8.9 -> 9.1, and 24 layers at n_kv 1024, 240
// workgroups into 192, 12.24 -> 14.13 us: those stay whole). Not for the
// matrix-core kernel, whose products cover 16 head columns whatever the chunk.
constexpr int64_t kDecodePartBytes = 128 << 10;

struct DecodePlan {
  int group = 1, n_chunks = 1;  // heads per chunk (the widest), chunks per KV head
  int n_wg = 0;    // workgroups with work (records)
  int grid_x = 0;  // the widest item's workgroups (grid rows are items)
  bool dyn = false;     // dynamic sub-tile claims
  bool long_waves = false;  // every wave streams 4 or more sub-tiles on average
  bool mf = false;      // matrix-core kernel
  bool stream = false;  // the streaming kernel (decode_stream.hip)
};

// The streaming kernel's plan: groups of up to 8 heads, kpg parts per group
// sized so that the launch has about one workgroup per CU (each part at least
// one sub-tile). Returns false where the kernel does not apply.
constexpr int kStreamWaves = 8;
bool plan_stream(DecodePlan& p, mi::DecodeItem* it, int n_items, int n_head_kv, int n_rep, int head_dim) {
  if (head_dim != 64 && head_dim != 128) return false;
  p = DecodePlan{};
  p.group = mi::decode_group_size(n_rep);
  p.n_chunks = mi::decode_chunks(n_rep);
  const int gpi = n_head_kv * p.n_chunks;
  int64_t sub = 0;
  for (int i = 0; i < n_items; ++i) {
    it[i].spg = (it[i].n_kv + mi::kDecodeSub - 1) / mi::kDecodeSub;
    sub += (int64_t)gpi * it[i].spg;
  }
  // Parts per group: about one workgroup per CU for the launch, at most
  // kStreamMaxParts (the last part to arrive merges every record, kStreamMaxParts
  // of them in two rounds of loads; one layer at n_kv 4096 took 63 us with 128
  // parts against 8 us for the ring kernel), each at least 4 sub-tiles.
  constexpr int64_t kStreamMaxParts = 16;
  int64_t wg = 0;
  for (int i = 0; i < n_items; ++i) {
    int64_t k = g.knobs.kpg > 0 ? g.knobs.kpg : (int64_t)g.n_cu * it[i].spg / std::max<int64_t>(1, sub);
    if (g.knobs.kpg <= 0) k = std::min<int64_t>(k, std::min<int64_t>(kStreamMaxParts, it[i].spg / 4));
    k = std::max<int64_t>(1, std::min<int64_t>(k, it[i].spg));
    it[i].kpg = (int32_t)k;
    it[i].wg0 = (int32_t)wg;
    wg += (int64_t)gpi * k;
    p.grid_x = std::max<int>(p.grid_x, gpi * (int)k);
  }
  p.n_wg = (int)wg;
  p.long_waves = sub >= (int64_t)g.knobs.stream_min * wg * kStreamWaves;
  p.stream = true;
  return true;
}

// Assigns kpg and the first record of every item for gpi groups per item.
// pos_bytes: one position's K and V row bytes.
void plan_items(DecodePlan& p, mi::DecodeItem* it, int n_items, int gpi, int waves, int ring, int pos_bytes) {
  int64_t sub = 0;
  for (int i = 0; i < n_items; ++i) {
    it[i].spg = (it[i].n_kv + mi::kDecodeSub - 1) / mi::kDecodeSub;
    sub += (int64_t)gpi * it[i].spg;
  }
  const int forced = g.knobs.kpg;
  int64_t wg = 0;
  p.dyn = false;
  p.grid_x = 0;
  for (int i = 0; i < n_items; ++i) {
    const int64_t cap = std::max<int64_t>(1, (it[i].spg + waves - 1) / waves);
    int64_t k = forced > 0 ? forced : (int64_t)g.n_cu * it[i].spg / std::max<int64_t>(1, sub);
    // Launches of few, long groups (merged by all parts, more than
    // kDecodeEarlyMax of them): no more parts than either half the CUs' share
    // or parts of kDecodePartBytes give, whichever is more. The merge costs
    // more per part than a part's extra streaming saves below that size: one
    // layer of 2 KV heads at n_kv 16384 (F32, D 64) 12.9 -> 11.9 us with 64
    // parts instead of 128, 28/4 heads, D 128, F16 at n_kv 4096 9.8 -> 9.2 us
    // with 32 instead of 64.
    if (forced <= 0 && k > mi::kDecodeEarlyMax) {
      const int64_t by_bytes = ((int64_t)it[i].spg * mi::kDecodeSub * pos_bytes + kDecodePartBytes - 1) /
                               kDecodePartBytes;
      k = std::min(k, std::max(by_bytes, k / 2));
    }
    if (forced <= 0 && it[i].spg <= (int64_t)g.knobs.solo * ring) k = 1;
    k = std::max<int64_t>(1, std::min<int64_t>(k, cap));
    it[i].kpg = (int32_t)k;
    it[i].wg0 = (int32_t)wg;
    wg += (int64_t)gpi * k;
    if (k > 1 && g.knobs.claim > 0 && it[i].spg >= (int64_t)g.knobs.claim * k * ring && !g.deterministic)
      p.dyn = true;
  }
  for (int i = 0; i < n_items; ++i) p.grid_x = std::max(p.grid_x, gpi * it[i].kpg);
  p.n_wg = (int)wg;
  p.long_waves = sub >= 4 * wg * waves;
}

// max_groups: the workspace's group capacity (a head split must fit in it).
DecodePlan plan_decode(mi::DecodeItem* it, int n_items, int n_head_kv, int n_rep, int head_dim,
                       bool f16, int max_groups) {
  DecodePlan p;
  p.group = mi::decode_group_size(n_rep);
  p.n_chunks = mi::decode_chunks(n_rep);
  const int waves = mi::decode_wg_waves(head_dim, f16);
  const int ring = waves * mi::decode_ring_slots(head_dim, f16);
  const int pos_bytes = 2 * head_dim * (f16 ? 2 : 4);
  plan_items(p, it, n_items, n_head_kv * p.n_chunks, waves, ring, pos_bytes);
  const int dmode = g.decode_mode.load();
  const bool autom = dmode == MI_HIP_DECODE_AUTO;
  // AUTO keeps an F32 cache on the vector units (float products, as the
  // reference's ops): the matrix form splits F32 operands into bf16 pairs,
  // whose ~2^-16 relative error per product grows with the score magnitude.
  p.mf = dmode == MI_HIP_DECODE_MATRIX;
  bool split = false;
  // Head split. hsplit 1: only when every group has one workgroup; 2: also
  // when groups merge parts, if the split launch keeps every item's parts
  // (its workgroups double, none streams more than before) within one
  // workgroup per CU.
  if (g.knobs.kpg <= 0 && g.knobs.hsplit && !p.mf && p.group > 4 &&
      (int64_t)n_items * n_head_kv * p.n_chunks * 2 <= max_groups) {
    int32_t kpg0[mi::kDecodeMaxItems];
    bool solo = true;
    for (int i = 0; i < n_items; ++i) {
      kpg0[i] = it[i].kpg;
      solo = solo && kpg0[i] == 1;
    }
    if (solo || (g.knobs.hsplit >= 2 && 2 * p.n_wg <= g.n_cu)) {
      DecodePlan q = p;
      q.group = (p.group + 1) / 2;
      q.n_chunks = p.n_chunks * 2;
      plan_items(q, it, n_items, n_head_kv * q.n_chunks, waves, ring, pos_bytes);
      bool keep = true;
      for (int i = 0; i < n_items; ++i) keep = keep && it[i].kpg >= kpg0[i];
      // An F16 cache takes the split (vector units) only where the split
      // launch's waves stream fewer than 4 sub-tiles each on average; longer
      // streams run faster whole on the matrix cores. One layer, F16, with the
      // split's sub-tiles per wave: 28/4 heads, D 128 at n_kv 8192 (4) 10.7
      // against 14.5 us split; 14/2 heads, D 64 at 32768 (4) 11.9 against
      // 14.3; at 8192 (2) 9.5 against 9.6; at 1024-4096 (1) 7.9-8.0 against
      // 9.0-9.1 split; 28/4 heads at 512 (1) 8.8 against 10.5 split.
      if (autom && f16 && q.long_waves) keep = false;
      if (keep) {
        q.mf = p.mf;  // sub-tiles and workgroups both double: long_waves stands
        p = q;
        split = true;
      } else {
        plan_items(p, it, n_items, n_head_kv * p.n_chunks, waves, ring, pos_bytes);
      }
    }
  }
  // An F16 cache runs on the vector units only where its heads were split
  // (above); otherwise on the matrix cores (24 layers of 14/2 heads at n_kv
  // 4096: 15.8 against 20.8 us).
  if (autom && f16 && !split) p.mf = true;
  return p;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace

// ---------------------------------------------------------------------------
// Decode workspace: [status words][two counter sets][records], each part
// 256-byte aligned. Zeroed once at creation; afterwards the kernels keep the
// counter sets zero between launches (see decode.hip) and the epoch stamps
// make stale records recognisable.
// ---------------------------------------------------------------------------
struct mi_hip_workspace {
  int groups = 0;           // groups one launch may have (counter-set capacity)
  size_t rec_bytes = 0;     // record capacity
  char* base = nullptr;
  size_t bytes = 0;
  unsigned* status = nullptr;
  unsigned* cnt = nullptr;
  float* rec = nullptr;
  std::mutex mu;
  uint32_t epoch = 0;       // stamp of the last launch
  int dirty[2] = {0, 0};    // counter set s: groups [0, dirty[s]) the last launch on it used
  int32_t max_polls = 4096;
  bool borrowed = false;    // memory not owned (never freed)
};

// Scratch of mi_hip_attn_decode_batch_noalloc: a decode workspace laid over a
// fixed device array (no allocation ever), one per GPU that loads this code
// object. Its name is only a host-side stand-in; the device address comes
// from hipGetSymbolAddress at mi_hip_init.
constexpr size_t kScratchBytes = 4u << 20;
constexpr int kScratchGroups = 128;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr size_t kWsAlign = 256;
size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

size_t ws_counter_bytes(int groups) { return 2 * (size_t)groups * mi::kCtrInts * sizeof(unsigned); }

// Bytes of a workspace covering `groups` groups and `rec_bytes` of records.
size_t ws_total_bytes(int groups, size_t rec_bytes) {
  return kWsAlign + round_up(ws_counter_bytes(groups), kWsAlign) + round_up(rec_bytes, kWsAlign);
}

// Lays a workspace over [base, base + bytes).
void ws_layout(mi_hip_workspace* ws, char* base, int groups, size_t rec_bytes) {
  ws->base = base;
  ws->groups = groups;
  ws->rec_bytes = rec_bytes;
  ws->bytes = ws_total_bytes(groups, rec_bytes);
  ws->status = reinterpret_cast<unsigned*>(base);
  ws->cnt = reinterpret_cast<unsigned*>(base + kWsAlign);
  ws->rec = reinterpret_cast<float*>(base + kWsAlign + round_up(ws_counter_bytes(groups), kWsAlign));
}

// Groups and record bytes that cover every decode launch of a head shape: up
// to kDecodeMaxItems items, at most one workgroup per CU plus one per group
// (the planner's at-least-one rounding), or the forced kpg.
void ws_capacity(int n_head_kv, int n_rep, int head_dim, int* groups, size_t* rec_bytes) {
  const int group = mi::decode_group_size(n_rep);
  // a head split doubles the groups (records stay: each holds half the heads)
  const int64_t gr = (int64_t)mi::kDecodeMaxItems * n_head_kv * mi::decode_chunks(n_rep) * (group > 4 ? 2 : 1);
  const int64_t wgs = g.knobs.kpg > 0 ? gr * g.knobs.kpg : g.n_cu + gr;
  *groups = (int)gr;
  *rec_bytes = (size_t)wgs * mi::decode_record_floats(head_dim, group) * sizeof(float);
}

int ws_create(int groups, size_t rec_bytes, mi_hip_workspace** out) {
  *out = nullptr;
  mi_hip_workspace* ws = new (std::nothrow) mi_hip_workspace();
  if (!ws) return fail(MI_HIP_E_NOMEM, "host allocation failed");
  void* p = nullptr;
  const size_t bytes = ws_total_bytes(groups, rec_bytes);
  int rc = dev_alloc(&p, bytes, "decode workspace");
  if (rc) {
    delete ws;
    return rc;
  }
  hipError_t e = hipMemset(p, 0, bytes);  // counters zero, record stamps 0 (no launch's epoch)
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    dev_free(p, bytes);
    delete ws;
    return hip_fail(e, "workspace init");
  }
  ws_layout(ws, static_cast<char*>(p), groups, rec_bytes);
  *out = ws;
  return MI_HIP_OK;
}

// The workspace over the static scratch array at device address `ptr`.
int ws_over_scratch(void* ptr, mi_hip_workspace** out) {
  *out = nullptr;
  mi_hip_workspace* ws = new (std::nothrow) mi_hip_workspace();
  if (!ws) return fail(MI_HIP_E_NOMEM, "host allocation failed");
  const size_t rec = kScratchBytes - (ws_total_bytes(kScratchGroups, 0) - 0);
  ws_layout(ws, static_cast<char*>(ptr), kScratchGroups, rec & ~(kWsAlign - 1));
  ws->borrowed = true;
  *out = ws;
  return MI_HIP_OK;
}

void ws_destroy(mi_hip_workspace* ws) {
  if (!ws) return;
  if (!ws->borrowed) dev_free(ws->base, ws->bytes);
  delete ws;
}

// The stamp of the next launch on ws, which uses `groups` groups: never 0 (the
// stamp of zeroed records), and alternating in parity (the counter sets).
// After 2^32 launches the stamps start again at 2 (even, after the odd
// 2^32 - 1), and the records are zeroed first so that no stale record can
// carry a reused stamp. *clear: the groups of the other set that the launch
// must clear (those the launch before it used).
int ws_next_epoch(mi_hip_workspace* ws, int groups, hipStream_t stream, uint32_t* epoch, int* clear) {
  std::lock_guard<std::mutex> lk(ws->mu);
  if (++ws->epoch == 0) {
    ws->epoch = 2;
    hipError_t e = mi::launch_fill_u32(reinterpret_cast<unsigned*>(ws->rec), ws->rec_bytes / 4, 0u, stream);
    if (e != hipSuccess) return hip_fail(e, "workspace record reset");
  }
  const int s = (int)(ws->epoch & 1u);
  *epoch = ws->epoch;
  *clear = ws->dirty[s ^ 1];
  ws->dirty[s ^ 1] = 0;
  ws->dirty[s] = groups;
  return MI_HIP_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// KV cache object
// ---------------------------------------------------------------------------
struct mi_hip_kv {
  mi_hip_workspace* ws = nullptr;  // its own decode workspace
  mi_hip_kv_desc d;
  char* base = nullptr;
  size_t bytes = 0;
  size_t tensor_bytes = 0;  // one layer's K (or V)
  int64_t s1 = 0, s2 = 0;   // byte strides: head, position
  int elt = 4;
  float* stage = nullptr;   // host-node staging: Q, O, appended rows
  size_t stage_bytes = 0;
  size_t q_floats = 0, row_floats = 0;
  hipStream_t stream = nullptr;

  char* tensor(int layer, int which) const {
    return base + (size_t)(2 * layer + which) * tensor_bytes;
  }
};

namespace {

struct Resolved {
  const char* k;
  const char* v;
  int64_t k_s1, k_s2, v_s1, v_s2;
  bool f16;
  int head_dim, n_head_kv;
  int n_ctx;  // -1 when unknown (explicit tensors)
};

int resolve_kv(const mi_hip_attn_args* a, Resolved* r) {
  if (a->kv) {
    const mi_hip_kv* kv = a->kv;
    if (a->layer < 0 || a->layer >= kv->d.n_layer)
      return fail(MI_HIP_E_INVALID, "layer %d out of range [0, %d)", a->layer, kv->d.n_layer);
    r->k = kv->tensor(a->layer, 0);
    r->v = kv->tensor(a->layer, 1);
    r->k_s1 = r->v_s1 = kv->s1;
    r->k_s2 = r->v_s2 = kv->s2;
    r->f16 = kv->d.type == MI_TYPE_F16;
    r->head_dim = kv->d.head_dim;
    r->n_head_kv = kv->d.n_head_kv;
    r->n_ctx = kv->d.n_ctx;
    return MI_HIP_OK;
  }
  if (!a->k || !a->v) return fail(MI_HIP_E_INVALID, "no KV source: kv and k/v are NULL");
  if (a->kv_type != MI_TYPE_F32 && a->kv_type != MI_TYPE_F16)
    return fail(MI_HIP_E_UNSUPPORTED, "K/V type %d: only F32 (0) and F16 (1)", a->kv_type);
  const int elt = a->kv_type == MI_TYPE_F16 ? 2 : 4;
  if (a->k_nb[0] != (size_t)elt || a->v_nb[0] != (size_t)elt)
    return fail(MI_HIP_E_UNSUPPORTED, "K/V nb[0] must be the element size (%d)", elt);
  const size_t al = (size_t)elt * 4;
  for (int i = 1; i < 3; ++i)
    if (a->k_nb[i] % al || a->v_nb[i] % al)
      return fail(MI_HIP_E_UNSUPPORTED, "K/V nb[1], nb[2] must be multiples of %zu bytes", al);
  if (!aligned(a->k, al) || !aligned(a->v, al))
    return fail(MI_HIP_E_UNSUPPORTED, "K/V data must be %zu-byte aligned", al);
  r->k = static_cast<const char*>(a->k);
  r->v = static_cast<const char*>(a->v);
  r->k_s1 = (int64_t)a->k_nb[1];
  r->k_s2 = (int64_t)a->k_nb[2];
  r->v_s1 = (int64_t)a->v_nb[1];
  r->v_s2 = (int64_t)a->v_nb[2];
  r->f16 = a->kv_type == MI_TYPE_F16;
  r->head_dim = a->head_dim;
  r->n_head_kv = a->n_head_kv;
  r->n_ctx = -1;
  return MI_HIP_OK;
}

// Checks everything the fused kernels assume about one problem.
int check_problem(const mi_hip_attn_args* a, const Resolved& r) {
  if (r.head_dim != 64 && r.head_dim != 128)
    return fail(MI_HIP_E_UNSUPPORTED, "head_dim %d: the kernels cover 64 and 128", r.head_dim);
  if (r.n_head_kv <= 0) return fail(MI_HIP_E_INVALID, "n_head_kv must be positive");
  if (a->n_rep <= 0 || a->n_head <= 0)
    return fail(MI_HIP_E_INVALID, "n_head (%d) and n_rep (%d) must be positive", a->n_head, a->n_rep);
  if (a->n_head != a->n_rep * r.n_head_kv)
    return fail(MI_HIP_E_INVALID, "n_head (%d) must equal n_rep (%d) * n_head_kv (%d)", a->n_head,
                a->n_rep, r.n_head_kv);
  if (a->n_past < 0 || a->n_tokens < 1)
    return fail(MI_HIP_E_INVALID, "n_past (%d) must be >= 0 and n_tokens (%d) >= 1", a->n_past,
                a->n_tokens);
  if (r.n_ctx >= 0 && (int64_t)a->n_past + a->n_tokens > r.n_ctx)
    return fail(MI_HIP_E_INVALID, "n_past + n_tokens (%d) exceeds n_ctx (%d)",
                a->n_past + a->n_tokens, r.n_ctx);
  if (!std::isfinite(a->scale)) return fail(MI_HIP_E_INVALID, "scale must be finite");
  if (!a->q || !a->out) return fail(MI_HIP_E_INVALID, "q and out must be device pointers");
  if (a->q_nb[0] != 4 || a->out_nb[0] != 4)
    return fail(MI_HIP_E_UNSUPPORTED, "q/out nb[0] must be 4 (head_dim contiguous)");
  for (int i = 1; i < 3; ++i)
    if (a->q_nb[i] % 16 || a->out_nb[i] % 16)
      return fail(MI_HIP_E_UNSUPPORTED, "q/out nb[1], nb[2] must be multiples of 16 bytes");
  if (!aligned(a->q, 16) || !aligned(a->out, 16))
    return fail(MI_HIP_E_UNSUPPORTED, "q/out must be 16-byte aligned");
  return MI_HIP_OK;
}

mi::DecodeItem make_item(const mi_hip_attn_args* a, const Resolved& r) {
  mi::DecodeItem it{};
  it.k = r.k;
  it.v = r.v;
  it.q = a->q;
  it.out = a->out;
  it.k_s1 = r.k_s1;
  it.k_s2 = r.k_s2;
  it.v_s1 = r.v_s1;
  it.v_s2 = r.v_s2;
  it.q_s1 = (int64_t)a->q_nb[1];
  it.o_s1 = (int64_t)a->out_nb[1];
  it.n_kv = a->n_past + 1;
  return it;
}

// The workspace a decode call uses: the first item's, else its cache's, else
// the library default.
mi_hip_workspace* workspace_of(const mi_hip_attn_args* a) {
  if (a->ws) return a->ws;
  if (a->kv) return a->kv->ws;
  return g.default_ws;
}

int run_decode(const mi_hip_attn_args* items, int n, hipStream_t stream, mi_hip_workspace* ws) {
  if (!ws) return fail(MI_HIP_E_STATE, "no decode workspace (the library default is gone)");
  // Each launch's stamp and counter-set parity are chosen here on the host
  // and passed by value, so a captured launch would replay stale ones.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  MI_TRY_HIP(hipStreamIsCapturing(stream, &cap), "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(MI_HIP_E_UNSUPPORTED,
                "decode launches cannot be captured into a graph (each launch takes a fresh stamp)");
  Resolved r0;
  int rc = resolve_kv(&items[0], &r0);
  if (rc) return rc;
  const int elt = r0.f16 ? 2 : 4;
  // Launches of up to kDecodeMaxItems consecutive items sharing the position
  // strides (the kernel's per-lane load offsets derive from them). Every
  // launch is planned and checked against the workspace before the first is
  // enqueued, so a refused call leaves no partial output behind.
  auto plan_launch = [&](int base, mi::DecodeParams& p, int& cnt, DecodePlan& plan) -> int {
    p = mi::DecodeParams{};
    cnt = 0;
    for (; cnt < mi::kDecodeMaxItems && base + cnt < n; ++cnt) {
      Resolved r;
      int rc2 = resolve_kv(&items[base + cnt], &r);
      if (rc2) return rc2;
      if (cnt > 0 && (r.k_s2 != p.item[0].k_s2 || r.v_s2 != p.item[0].v_s2)) break;
      if (r.k_s2 < (int64_t)r.head_dim * elt || r.v_s2 < (int64_t)r.head_dim * elt)
        return fail(MI_HIP_E_UNSUPPORTED, "item %d: position stride below one row", base + cnt);
      p.item[cnt] = make_item(&items[base + cnt], r);
      // one group's rows are addressed with 32-bit byte offsets
      const int64_t last = (int64_t)(p.item[cnt].n_kv - 1);
      if (last * r.k_s2 + (int64_t)r.head_dim * elt > INT32_MAX ||
          last * r.v_s2 + (int64_t)r.head_dim * elt > INT32_MAX)
        return fail(MI_HIP_E_UNSUPPORTED,
                    "item %d: n_kv * position stride exceeds 2^31 bytes for one KV head", base + cnt);
    }
    const int dmode = g.decode_mode.load();
    bool streamed = false;
    if (dmode == MI_HIP_DECODE_STREAM || (dmode == MI_HIP_DECODE_AUTO && g.knobs.stream_min > 0 && !r0.f16)) {
      DecodePlan sp;
      if (plan_stream(sp, p.item, cnt, r0.n_head_kv, items[0].n_rep, r0.head_dim) &&
          (dmode == MI_HIP_DECODE_STREAM || sp.long_waves)) {
        plan = sp;
        streamed = true;
      }
    }
    if (!streamed) plan = plan_decode(p.item, cnt, r0.n_head_kv, items[0].n_rep, r0.head_dim, r0.f16, ws->groups);
    const int gpi = r0.n_head_kv * plan.n_chunks;
    const int team = mi::decode_team(r0.head_dim, r0.f16, plan.group);
    for (int i = 0; i < cnt; ++i)
      if ((p.item[i].kpg + team - 1) / team > 64 - mi::kCtrTeams)
        return fail(MI_HIP_E_UNSUPPORTED, "item %d: %d workgroups per group exceed the merge teams",
                    base + i, (int)p.item[i].kpg);
    const size_t rec_bytes =
        (size_t)plan.n_wg * mi::decode_record_floats(r0.head_dim, plan.group) * sizeof(float);
    if (cnt * gpi > ws->groups || rec_bytes > ws->rec_bytes)
      return fail(MI_HIP_E_UNSUPPORTED,
                  "decode launch of %d groups and %zu record bytes exceeds its workspace (%d groups, "
                  "%zu bytes): create the workspace for this head shape",
                  cnt * gpi, rec_bytes, ws->groups, ws->rec_bytes);
    p.n_rep = items[0].n_rep;
    p.n_head_kv = r0.n_head_kv;
    p.n_chunks = plan.n_chunks;
    p.gpi = gpi;
    p.n_wg = plan.n_wg;
    p.scale_log2e = items[0].scale * kLog2e;
    p.rec = ws->rec;
    p.cnt = ws->cnt;
    p.status = ws->status;
    p.ctr_groups = ws->groups;
    p.max_polls = ws->max_polls;
    p.rec_words = (int32_t)(mi::decode_record_floats(r0.head_dim, plan.group) / 2);
    p.det = g.deterministic.load();
    // The early merge is worth its wait when every workgroup of the launch can
    // be resident at once (one per CU); it stays correct otherwise.
    // (knob 2 forces it: tests of the fallback for parts that start late).
    p.early = g.knobs.early == 2 || (plan.n_wg <= g.n_cu && g.knobs.early != 0);
    return MI_HIP_OK;
  };
  mi::DecodeParams p;
  DecodePlan plan;
  int cnt = 0, launches = 0;
  for (int base = 0; base < n; base += cnt, ++launches)
    if ((rc = plan_launch(base, p, cnt, plan))) return rc;
  for (int base = 0; base < n; base += cnt) {
    // (a single launch is still planned in p)
    if (launches > 1 && (rc = plan_launch(base, p, cnt, plan))) return rc;
    if ((rc = ws_next_epoch(ws, cnt * p.gpi, stream, &p.epoch, &p.clear_groups))) return rc;
    hipError_t e =
        plan.stream
            ? mi::launch_stream_decode(p, plan.grid_x, cnt, r0.head_dim, r0.f16, plan.group, stream)
            : mi::launch_decode(p, plan.grid_x, cnt, r0.head_dim, r0.f16, plan.group, plan.dyn, plan.mf, stream);
    if (e != hipSuccess) return hip_fail(e, "decode launch");
  }
  return MI_HIP_OK;
}

// Whether a prefill runs the split product form: asked for, or (AUTO) with an
// F16 cache, whose f16 products are exact in the cache operand.
bool prefill_split(bool f16) {
  const int mode = g.prefill_mode.load();
  return mode == MI_HIP_PREFILL_SPLIT_BF16 || (mode == MI_HIP_PREFILL_AUTO && f16);
}

int run_prefill(const mi_hip_attn_args* a, const Resolved& r, hipStream_t stream) {
  // a KV head's rows, up to the last key tile's end, are addressed with 32-bit
  // byte offsets
  const int64_t rows = (int64_t)a->n_past + a->n_tokens + mi::kPrefillKeys;
  const int64_t row_bytes = (int64_t)r.head_dim * (r.f16 ? 2 : 4);
  if (rows * r.k_s2 + row_bytes > INT32_MAX || rows * r.v_s2 + row_bytes > INT32_MAX)
    return fail(MI_HIP_E_UNSUPPORTED, "n_kv * position stride exceeds 2^31 bytes for one KV head");
  // rows past n_kv must lie past the range the kernel's loads are bounded by
  if (r.k_s2 < row_bytes || r.v_s2 < row_bytes)
    return fail(MI_HIP_E_UNSUPPORTED, "K/V position stride below one row");
  mi::PrefillParams p{};
  p.k = r.k;
  p.v = r.v;
  p.q = a->q;
  p.out = a->out;
  p.k_s1 = r.k_s1;
  p.k_s2 = r.k_s2;
  p.v_s1 = r.v_s1;
  p.v_s2 = r.v_s2;
  p.q_s1 = (int64_t)a->q_nb[1];
  p.q_s2 = (int64_t)a->q_nb[2];
  p.o_s1 = (int64_t)a->out_nb[1];
  p.o_s2 = (int64_t)a->out_nb[2];
  p.n_head = a->n_head;
  p.n_rep = a->n_rep;
  p.n_past = a->n_past;
  p.n_tokens = a->n_tokens;
  p.n_qblocks = (a->n_tokens + mi::kPrefillRows - 1) / mi::kPrefillRows;
  p.scale_log2e = a->scale * kLog2e;
  p.det = g.deterministic.load();
  hipError_t e = mi::launch_prefill(p, r.head_dim, r.f16, g.n_cu,
                                    prefill_split(r.f16), stream);
  if (e != hipSuccess) return hip_fail(e, "prefill launch");
  return MI_HIP_OK;
}

// ---------------------------------------------------------------------------
// Executor hook tables (no allocation per step)
// ---------------------------------------------------------------------------
struct Binding {
  mi_hip_kv* kv;
  int layer;
  int which;
};
std::mutex g_bind_mu;
std::unordered_map<const mi_tensor*, Binding> g_bind;

const Binding* find_binding(const mi_tensor* t) {
  if (!t) return nullptr;
  std::lock_guard<std::mutex> lk(g_bind_mu);
  auto it = g_bind.find(t);
  return it == g_bind.end() ? nullptr : &it->second;
}

// Fixed-capacity pointer map, cleared in O(1) by bumping a generation.
template <int N>
struct PtrMap {
  struct Slot {
    const void* key;
    uint32_t gen;
    int32_t val;
  };
  Slot slot[N];
  uint32_t gen = 1;
  void clear() { ++gen; }
  static uint32_t hash(const void* p) {
    uint64_t x = reinterpret_cast<uintptr_t>(p);
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdULL;
    x ^= x >> 33;
    return (uint32_t)x;
  }
  int32_t* find(const void* key, bool insert) {
    uint32_t h = hash(key) & (N - 1);
    for (int probe = 0; probe < N; ++probe, h = (h + 1) & (N - 1)) {
      Slot& s = slot[h];
      if (s.gen != gen) {
        if (!insert) return nullptr;
        s.key = key;
        s.gen = gen;
        s.val = 0;
        return &s.val;
      }
      if (s.key == key) return &s.val;
    }
    return nullptr;
  }
};

enum Role : int32_t { kNone = 0, kFusedQK = 1, kFusedSoftmax = 2, kFusedKQV = 3 };

std::mutex g_plan_mu;
PtrMap<1 << 15> g_readers;  // ATTN_QK / SOFTMAX node -> number of readers
PtrMap<1 << 15> g_roles;    // node -> Role

int32_t role_of(const mi_tensor* t) {
  std::lock_guard<std::mutex> lk(g_plan_mu);
  int32_t* r = g_roles.find(t, false);
  return r ? *r : kNone;
}

bool contiguous3(const mi_tensor* t) {
  return t->nb[0] == 4 && t->nb[1] == 4 * (size_t)t->ne[0] &&
         t->nb[2] == t->nb[1] * (size_t)t->ne[1];
}

mi::NodeView view_of(const mi_tensor* t) {
  mi::NodeView v;
  v.data = static_cast<char*>(t->data);
  for (int i = 0; i < 3; ++i) {
    v.ne[i] = t->ne[i];
    v.nb[i] = (int64_t)t->nb[i];
  }
  return v;
}

int check_kv_tensor(const mi_tensor* t, const char* what) {
  if (!t || !t->data) return fail(MI_HIP_E_INVALID, "%s: missing tensor or data", what);
  if (t->type != MI_TYPE_F32 && t->type != MI_TYPE_F16)
    return fail(MI_HIP_E_UNSUPPORTED, "%s: type %d (F32 or F16 only)", what, (int)t->type);
  if (t->nb[0] != (t->type == MI_TYPE_F16 ? 2u : 4u))
    return fail(MI_HIP_E_UNSUPPORTED, "%s: nb[0] must be the element size", what);
  return MI_HIP_OK;
}

int check_f32(const mi_tensor* t, const char* what) {
  if (!t || !t->data) return fail(MI_HIP_E_INVALID, "%s: missing tensor or data", what);
  if (t->type != MI_TYPE_F32) return fail(MI_HIP_E_UNSUPPORTED, "%s: must be F32", what);
  return MI_HIP_OK;
}

// Fills args for the fused chain ending at ATTN_KQV node `kqv`, all tensors
// device-resident.
int fused_args_from_nodes(mi_tensor* kqv, mi_hip_attn_args* a) {
  if (!kqv || kqv->op != MI_OP_ATTN_KQV) return fail(MI_HIP_E_INVALID, "dst is not an ATTN_KQV node");
  const mi_tensor* sm = kqv->src[0];
  if (!sm || sm->op != MI_OP_SOFTMAX) return fail(MI_HIP_E_INVALID, "ATTN_KQV src[0] is not SOFTMAX");
  const mi_tensor* qk = sm->src[0];
  if (!qk || qk->op != MI_OP_ATTN_QK) return fail(MI_HIP_E_INVALID, "SOFTMAX src[0] is not ATTN_QK");
  const mi_tensor* q = qk->src[0];
  const mi_tensor* k = qk->src[1];
  const mi_tensor* v = kqv->src[1];
  int rc;
  if ((rc = check_f32(q, "Q")) || (rc = check_kv_tensor(k, "K")) || (rc = check_kv_tensor(v, "V")) ||
      (rc = check_f32(kqv, "out")))
    return rc;
  if (k->type != v->type) return fail(MI_HIP_E_UNSUPPORTED, "K and V types differ");
  const int n_past = mi_tensor_param_i32(qk, 0);
  const int n_rep = mi_tensor_param_i32(qk, 1);
  if (mi_tensor_param_i32(sm, 0) != n_past)
    return fail(MI_HIP_E_INVALID, "SOFTMAX n_past differs from ATTN_QK n_past");
  if (mi_tensor_param_i32(kqv, 0) != n_rep)
    return fail(MI_HIP_E_INVALID, "ATTN_KQV n_rep differs from ATTN_QK n_rep");
  if (qk->ne[0] != (int64_t)n_past + q->ne[2] || qk->ne[1] != q->ne[2] || qk->ne[2] != q->ne[1])
    return fail(MI_HIP_E_INVALID, "ATTN_QK shape is not [n_past+n_tokens, n_tokens, n_head]");
  if (kqv->ne[0] != q->ne[0] || kqv->ne[1] != q->ne[1] || kqv->ne[2] != q->ne[2])
    return fail(MI_HIP_E_INVALID, "ATTN_KQV shape is not [head_dim, n_head, n_tokens]");
  if (k->ne[0] != q->ne[0] || v->ne[0] != q->ne[0] || k->ne[1] != v->ne[1])
    return fail(MI_HIP_E_INVALID, "K/V head_dim or n_head_kv mismatch");
  if (k->ne[2] < qk->ne[0] || v->ne[2] < qk->ne[0])
    return fail(MI_HIP_E_INVALID, "K/V hold fewer than n_past + n_tokens positions");
  std::memset(a, 0, sizeof *a);
  a->k = k->data;
  a->v = v->data;
  for (int i = 0; i < 3; ++i) {
    a->k_nb[i] = k->nb[i];
    a->v_nb[i] = v->nb[i];
    a->q_nb[i] = q->nb[i];
    a->out_nb[i] = kqv->nb[i];
  }
  a->kv_type = k->type;
  a->head_dim = (int32_t)q->ne[0];
  a->n_head_kv = (int32_t)k->ne[1];
  a->q = static_cast<const float*>(q->data);
  a->out = static_cast<float*>(kqv->data);
  a->n_head = (int32_t)q->ne[1];
  a->n_rep = n_rep;
  a->n_past = n_past;
  a->n_tokens = (int32_t)q->ne[2];
  a->scale = mi_tensor_param_f32(sm, 1);
  return MI_HIP_OK;
}

}  // namespace

namespace mi {
int rt_fail(int code, const char* msg) { return fail(code, "%s", msg); }
int rt_hip_fail(hipError_t e, const char* what) { return hip_fail(e, what); }
int rt_alloc(void** p, size_t bytes, const char* what) { return dev_alloc(p, bytes, what); }
void rt_free(void* p, size_t bytes) { dev_free(p, bytes); }
int rt_bind() { return bind_device(); }
int rt_n_cu() { return g.n_cu; }
}  // namespace mi

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

int mi_hip_init(int device) {
  std::lock_guard<std::mutex> lk(g.mu);
  if (g.ready) {
    if (device == g.device) return MI_HIP_OK;
    return fail(MI_HIP_E_STATE, "already initialised on device %d", g.device);
  }
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return fail(MI_HIP_E_NODEVICE, "no HIP device is visible");
  if (device < 0 || device >= n)
    return fail(MI_HIP_E_INVALID, "device %d out of range [0, %d)", device, n);
  hipDeviceProp_t prop;
  MI_TRY_HIP(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MI_HIP_E_NODEVICE, "device %d is %s; this library is built for gfx950 only", device,
                prop.gcnArchName);
  MI_TRY_HIP(hipSetDevice(device), "hipSetDevice");
  g.device = device;
  g.n_cu = prop.multiProcessorCount;
  g.knobs.kpg = env_int("MI_HIP_DECODE_KPG", 0);
  g.knobs.early = env_int("MI_HIP_DECODE_EARLY", 1);
  g.knobs.solo = env_int("MI_HIP_DECODE_SOLO", 1);
  g.knobs.claim = env_int("MI_HIP_DECODE_CLAIM", 0);
  g.knobs.hsplit = env_int("MI_HIP_DECODE_HSPLIT", 2);
  g.knobs.stream_min = env_int("MI_HIP_DECODE_STREAM_MIN", 0);
  g.ready = true;
  // The default workspace: head_dim up to 128, groups of up to 8 heads, up to
  // 1024 groups per launch (e.g. 32 items x 32 KV heads), ~11 MB.
  const int groups = 1024;
  const size_t rec = (size_t)(g.n_cu + groups) * mi::decode_record_floats(128, 8) * sizeof(float);
  int rc = ws_create(groups, rec, &g.default_ws);
  if (rc) {
    g.ready = false;
    return rc;
  }
  // The no-allocation entry point's scratch: this device's copy of the static
  // array (zero at load, as its counters and record stamps must start). Its
  // workspace is made once per device and never destroyed (a later session
  // continues its stamps over the records the array still holds).
  if (device >= kMaxDevices) {
    ws_destroy(g.default_ws);
    g.default_ws = nullptr;
    g.ready = false;
    return fail(MI_HIP_E_UNSUPPORTED, "device %d: at most %d devices", device, kMaxDevices);
  }
  if (!scratch_by_device[device]) {
    void* sp = nullptr;
    hipError_t se = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (se != hipSuccess || !sp) {
      ws_destroy(g.default_ws);
      g.default_ws = nullptr;
      g.ready = false;
      return hip_fail(se != hipSuccess ? se : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
    }
    if ((rc = ws_over_scratch(sp, &scratch_by_device[device]))) {
      ws_destroy(g.default_ws);
      g.default_ws = nullptr;
      g.ready = false;
      return rc;
    }
  }
  g.scratch_ws = scratch_by_device[device];
  t_err[0] = '\0';
  return MI_HIP_OK;
}

int mi_hip_shutdown(void) {
  if (!g.ready) return MI_HIP_OK;
  int rc = bind_device();
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g.mu);
  (void)hipDeviceSynchronize();
  ws_destroy(g.default_ws);
  g.default_ws = nullptr;
  g.scratch_ws = nullptr;  // kept in scratch_by_device, as the array keeps its contents
  {
    std::lock_guard<std::mutex> nl(g.node_mu);
    dev_free(g.node_stage, g.node_stage_bytes);
    g.node_stage = nullptr;
    g.node_stage_bytes = 0;
    if (g.node_stream) (void)hipStreamDestroy(g.node_stream);
    g.node_stream = nullptr;
  }
  g.ready = false;
  g.device = -1;
  return MI_HIP_OK;
}

const char* mi_hip_last_error(void) { return t_err; }

int mi_hip_abi_layout(size_t* out, int n) {
  if (!out || n < 15) return fail(MI_HIP_E_INVALID, "need an array of at least 15 entries");
  out[0] = sizeof(mi_tensor);
  out[1] = offsetof(mi_tensor, type);
  out[2] = offsetof(mi_tensor, ne);
  out[3] = offsetof(mi_tensor, nb);
  out[4] = offsetof(mi_tensor, op);
  out[5] = offsetof(mi_tensor, op_params);
  out[6] = offsetof(mi_tensor, src);
  out[7] = offsetof(mi_tensor, data);
  out[8] = offsetof(mi_tensor, view_src);
  out[9] = offsetof(mi_tensor, view_offs);
  out[10] = offsetof(mi_tensor, n_children);
  out[11] = offsetof(mi_tensor, flags);
  out[12] = offsetof(mi_tensor, name);
  out[13] = offsetof(mi_tensor, extra);
  out[14] = sizeof(mi_cgraph);
  return MI_HIP_OK;
}

int mi_hip_get_alloc_stats(mi_hip_alloc_stats* out) {
  if (!out) return fail(MI_HIP_E_INVALID, "out is NULL");
  out->n_malloc = g.n_malloc.load();
  out->n_free = g.n_free.load();
  out->bytes_live = g.live.load();
  out->bytes_peak = g.peak.load();
  return MI_HIP_OK;
}

int mi_hip_set_alloc_limit(uint64_t bytes) {
  g.limit.store(bytes);
  return MI_HIP_OK;
}

int mi_hip_kv_create(const mi_hip_kv_desc* d, mi_hip_kv** out) {
  if (!d || !out) return fail(MI_HIP_E_INVALID, "desc and out must be non-NULL");
  *out = nullptr;
  if (d->n_layer <= 0 || d->n_ctx <= 0 || d->n_head_kv <= 0 || d->n_head <= 0)
    return fail(MI_HIP_E_INVALID, "n_layer, n_ctx, n_head_kv and n_head must be positive");
  if (d->n_head % d->n_head_kv != 0)
    return fail(MI_HIP_E_INVALID, "n_head (%d) must be a multiple of n_head_kv (%d)", d->n_head,
                d->n_head_kv);
  if (d->head_dim != 64 && d->head_dim != 128)
    return fail(MI_HIP_E_UNSUPPORTED, "head_dim %d: the kernels cover 64 and 128", d->head_dim);
  if (d->type != MI_TYPE_F32 && d->type != MI_TYPE_F16)
    return fail(MI_HIP_E_UNSUPPORTED, "cache type %d: F32 (0) or F16 (1)", d->type);
  int rc = bind_device();
  if (rc) return rc;

  mi_hip_kv* kv = new (std::nothrow) mi_hip_kv();
  if (!kv) return fail(MI_HIP_E_NOMEM, "host allocation failed");
  kv->d = *d;
  kv->elt = d->type == MI_TYPE_F16 ? 2 : 4;
  kv->s1 = (int64_t)d->head_dim * kv->elt;
  kv->s2 = kv->s1 * d->n_head_kv;
  kv->tensor_bytes = (size_t)kv->s2 * d->n_ctx;
  kv->bytes = kv->tensor_bytes * 2 * d->n_layer;
  kv->q_floats = (size_t)d->n_ctx * d->n_head * d->head_dim;
  kv->row_floats = (size_t)d->n_ctx * d->n_head_kv * d->head_dim;
  kv->stage_bytes = (2 * kv->q_floats + kv->row_floats) * sizeof(float);

  void* p = nullptr;
  if ((rc = dev_alloc(&p, kv->bytes, "KV cache"))) {
    delete kv;
    return rc;
  }
  kv->base = static_cast<char*>(p);
  if ((rc = dev_alloc(&p, kv->stage_bytes, "KV staging"))) {
    dev_free(kv->base, kv->bytes);
    delete kv;
    return rc;
  }
  kv->stage = static_cast<float*>(p);
  hipError_t e = hipMemset(kv->base, 0, kv->bytes);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&kv->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    dev_free(kv->stage, kv->stage_bytes);
    dev_free(kv->base, kv->bytes);
    delete kv;
    return hip_fail(e, "KV cache init");
  }
  int groups;
  size_t rec_bytes;
  ws_capacity(d->n_head_kv, d->n_head / d->n_head_kv, d->head_dim, &groups, &rec_bytes);
  if ((rc = ws_create(groups, rec_bytes, &kv->ws))) {
    (void)hipStreamDestroy(kv->stream);
    dev_free(kv->stage, kv->stage_bytes);
    dev_free(kv->base, kv->bytes);
    delete kv;
    return rc;
  }
  *out = kv;
  return MI_HIP_OK;
}

int mi_hip_kv_destroy(mi_hip_kv* kv) {
  if (!kv) return MI_HIP_OK;
  int rc = bind_device();
  if (rc) return rc;
  {
    std::lock_guard<std::mutex> lk(g_bind_mu);
    for (auto it = g_bind.begin(); it != g_bind.end();)
      it = it->second.kv == kv ? g_bind.erase(it) : std::next(it);
  }
  (void)hipStreamSynchronize(kv->stream);
  (void)hipStreamDestroy(kv->stream);
  (void)hipDeviceSynchronize();  // no decode launch on another stream still uses the workspace
  ws_destroy(kv->ws);
  dev_free(kv->stage, kv->stage_bytes);
  dev_free(kv->base, kv->bytes);
  delete kv;
  return MI_HIP_OK;
}

int mi_hip_kv_workspace(mi_hip_kv* kv, mi_hip_workspace** out) {
  if (!kv || !out) return fail(MI_HIP_E_INVALID, "kv and out must be non-NULL");
  *out = kv->ws;
  return MI_HIP_OK;
}

int mi_hip_workspace_create(const mi_hip_workspace_desc* d, mi_hip_workspace** out) {
  if (!d || !out) return fail(MI_HIP_E_INVALID, "desc and out must be non-NULL");
  *out = nullptr;
  if (d->n_head_kv <= 0 || d->n_head <= 0 || d->n_head % d->n_head_kv != 0)
    return fail(MI_HIP_E_INVALID, "n_head (%d) must be a positive multiple of n_head_kv (%d)",
                d->n_head, d->n_head_kv);
  if (d->head_dim != 64 && d->head_dim != 128)
    return fail(MI_HIP_E_UNSUPPORTED, "head_dim %d: the kernels cover 64 and 128", d->head_dim);
  int rc = bind_device();
  if (rc) return rc;
  int groups;
  size_t rec_bytes;
  ws_capacity(d->n_head_kv, d->n_head / d->n_head_kv, d->head_dim, &groups, &rec_bytes);
  return ws_create(groups, rec_bytes, out);
}

int mi_hip_workspace_destroy(mi_hip_workspace* ws) {
  if (!ws) return MI_HIP_OK;
  int rc = bind_device();
  if (rc) return rc;
  if (ws == g.default_ws) return fail(MI_HIP_E_INVALID, "the default workspace belongs to the library");
  (void)hipDeviceSynchronize();
  ws_destroy(ws);
  return MI_HIP_OK;
}

int mi_hip_decode_tuning(int32_t kpg, int32_t early, int32_t solo, int32_t claim) {
  if (!g.ready) return fail(MI_HIP_E_STATE, "mi_hip_init has not been called");
  std::lock_guard<std::mutex> lk(g.mu);
  if (kpg >= 0) g.knobs.kpg = kpg;
  if (early >= 0) g.knobs.early = early;
  if (solo >= 0) g.knobs.solo = solo;
  if (claim >= 0) g.knobs.claim = claim;
  return MI_HIP_OK;
}

int mi_hip_set_prefill_mode(int32_t mode) {
  if (mode != MI_HIP_PREFILL_F32 && mode != MI_HIP_PREFILL_SPLIT_BF16 && mode != MI_HIP_PREFILL_AUTO)
    return fail(MI_HIP_E_INVALID,
                "prefill mode %d: MI_HIP_PREFILL_F32 (0), MI_HIP_PREFILL_SPLIT_BF16 (1) or MI_HIP_PREFILL_AUTO (2)",
                mode);
  g.prefill_mode.store(mode);
  return MI_HIP_OK;
}

int mi_hip_set_decode_mode(int32_t mode) {
  if (mode != MI_HIP_DECODE_VALU && mode != MI_HIP_DECODE_MATRIX && mode != MI_HIP_DECODE_AUTO &&
      mode != MI_HIP_DECODE_STREAM)
    return fail(MI_HIP_E_INVALID, "decode mode %d: MI_HIP_DECODE_VALU (0), _MATRIX (1), _AUTO (2) or _STREAM (3)",
                mode);
  g.decode_mode.store(mode);
  return MI_HIP_OK;
}

int mi_hip_set_deterministic(int32_t on) {
  if (on != 0 && on != 1) return fail(MI_HIP_E_INVALID, "on must be 0 or 1");
  g.deterministic.store(on);
  return MI_HIP_OK;
}

int mi_hip_workspace_set_poll_limit(mi_hip_workspace* ws, int32_t rounds) {
  if (!ws || rounds < 0) return fail(MI_HIP_E_INVALID, "ws must be non-NULL and rounds >= 0");
  std::lock_guard<std::mutex> lk(ws->mu);
  ws->max_polls = rounds;
  return MI_HIP_OK;
}

int mi_hip_workspace_check(mi_hip_workspace* ws, void* stream, mi_hip_workspace_status* out) {
  if (!ws) return fail(MI_HIP_E_INVALID, "ws is NULL");
  int rc = bind_device();
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  unsigned words[mi::kStatusWords] = {0, 0, 0, 0};
  MI_TRY_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
  MI_TRY_HIP(hipMemcpyAsync(words, ws->status, sizeof words, hipMemcpyDeviceToHost, st), "status copy");
  MI_TRY_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
  hipError_t e = mi::launch_fill_u32(ws->status, mi::kStatusWords, 0u, st);
  // A lost record leaves its group's counters wherever they stopped: start over.
  if (e == hipSuccess && words[1] != 0) {
    e = mi::launch_fill_u32(ws->cnt, ws_counter_bytes(ws->groups) / sizeof(unsigned), 0u, st);
    std::lock_guard<std::mutex> lk(ws->mu);
    ws->dirty[0] = ws->dirty[1] = 0;
  }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) return hip_fail(e, "workspace status reset");
  if (out) {
    out->early_fallbacks = words[0];
    out->lost_groups = words[1];
  }
  if (words[1] != 0) return fail(MI_HIP_E_LOST, "%u decode group(s) lost a record; outputs of those launches are NaN", words[1]);
  return MI_HIP_OK;
}

int mi_hip_kv_view(mi_hip_kv* kv, int layer, int which, void** data, int64_t ne[4], size_t nb[4]) {
  if (!kv || !data) return fail(MI_HIP_E_INVALID, "kv and data must be non-NULL");
  if (layer < 0 || layer >= kv->d.n_layer || (which != 0 && which != 1))
    return fail(MI_HIP_E_INVALID, "layer %d / which %d out of range", layer, which);
  *data = kv->tensor(layer, which);
  if (ne) {
    ne[0] = kv->d.head_dim;
    ne[1] = kv->d.n_head_kv;
    ne[2] = kv->d.n_ctx;
    ne[3] = 1;
  }
  if (nb) {
    nb[0] = (size_t)kv->elt;
    nb[1] = (size_t)kv->s1;
    nb[2] = (size_t)kv->s2;
    nb[3] = (size_t)kv->s2 * kv->d.n_ctx;
  }
  return MI_HIP_OK;
}

int mi_hip_kv_write(mi_hip_kv* kv, int layer, int which, int pos0, int n_tokens, const float* src,
                    const size_t src_nb[3], int src_on_device, void* stream) {
  if (!kv || !src || !src_nb) return fail(MI_HIP_E_INVALID, "kv, src and src_nb must be non-NULL");
  if (layer < 0 || layer >= kv->d.n_layer || (which != 0 && which != 1))
    return fail(MI_HIP_E_INVALID, "layer %d / which %d out of range", layer, which);
  if (pos0 < 0 || n_tokens < 0 || (int64_t)pos0 + n_tokens > kv->d.n_ctx)
    return fail(MI_HIP_E_INVALID, "positions [%d, %d) outside [0, %d)", pos0, pos0 + n_tokens,
                kv->d.n_ctx);
  if (src_nb[0] % 4 || src_nb[1] % 4 || src_nb[2] % 4)
    return fail(MI_HIP_E_INVALID, "src strides must be multiples of 4 bytes");
  if (n_tokens == 0) return MI_HIP_OK;
  int rc = bind_device();
  if (rc) return rc;
  hipStream_t st = stream ? static_cast<hipStream_t>(stream) : nullptr;
  char* dst = kv->tensor(layer, which);
  const int D = kv->d.head_dim, H = kv->d.n_head_kv;
  const bool src_contig = src_nb[0] == 4 && src_nb[1] == 4u * D && src_nb[2] == 4u * D * H;
  const char* dev_src = reinterpret_cast<const char*>(src);
  int64_t nb[3] = {(int64_t)src_nb[0], (int64_t)src_nb[1], (int64_t)src_nb[2]};
  if (!src_on_device) {
    // Host rows: one contiguous copy straight into an F32 cache, else via staging.
    const size_t bytes = (size_t)n_tokens * D * H * sizeof(float);
    if (src_contig && kv->elt == 4) {
      MI_TRY_HIP(hipMemcpyAsync(dst + (size_t)pos0 * kv->s2, src, bytes, hipMemcpyHostToDevice, st),
                 "hipMemcpyAsync(K/V rows)");
      MI_TRY_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
      return MI_HIP_OK;
    }
    if (!src_contig) return fail(MI_HIP_E_UNSUPPORTED, "host K/V rows must be contiguous");
    float* stage_rows = kv->stage + 2 * kv->q_floats;
    MI_TRY_HIP(hipMemcpyAsync(stage_rows, src, bytes, hipMemcpyHostToDevice, st),
               "hipMemcpyAsync(K/V rows)");
    dev_src = reinterpret_cast<const char*>(stage_rows);
    nb[0] = 4;
    nb[1] = 4LL * D;
    nb[2] = 4LL * D * H;
  }
  hipError_t e = mi::launch_kv_append(dst, kv->s1, kv->s2, kv->elt == 2, dev_src, nb, D, H, pos0,
                                      n_tokens, st);
  if (e != hipSuccess) return hip_fail(e, "kv append launch");
  if (!src_on_device) MI_TRY_HIP(hipStreamSynchronize(st), "hipStreamSynchronize");
  return MI_HIP_OK;
}

int mi_hip_kv_bind(mi_hip_kv* kv, int layer, int which, const mi_tensor* host_kv) {
  if (!kv || !host_kv) return fail(MI_HIP_E_INVALID, "kv and host_kv must be non-NULL");
  if (layer < 0 || layer >= kv->d.n_layer || (which != 0 && which != 1))
    return fail(MI_HIP_E_INVALID, "layer %d / which %d out of range", layer, which);
  if (host_kv->ne[0] != kv->d.head_dim || host_kv->ne[1] != kv->d.n_head_kv ||
      host_kv->ne[2] > kv->d.n_ctx)
    return fail(MI_HIP_E_INVALID, "host tensor shape does not match the cache");
  std::lock_guard<std::mutex> lk(g_bind_mu);
  g_bind[host_kv] = Binding{kv, layer, which};
  return MI_HIP_OK;
}

int mi_hip_attn_fwd(const mi_hip_attn_args* a) {
  if (!a) return fail(MI_HIP_E_INVALID, "args is NULL");
  Resolved r;
  int rc = resolve_kv(a, &r);
  if (rc) return rc;
  if ((rc = check_problem(a, r))) return rc;
  if ((rc = bind_device())) return rc;
  hipStream_t st = static_cast<hipStream_t>(a->stream);
  return a->n_tokens == 1 ? run_decode(a, 1, st, workspace_of(a)) : run_prefill(a, r, st);
}

int mi_hip_attn_fwd_reference_order(const mi_hip_attn_args* a) {
  if (!a) return fail(MI_HIP_E_INVALID, "args is NULL");
  Resolved r;
  int rc = resolve_kv(a, &r);
  if (rc) return rc;
  if ((rc = check_problem(a, r))) return rc;
  if (r.f16) return fail(MI_HIP_E_UNSUPPORTED, "reference-order attention reads an F32 cache (the reference's)");
  const int64_t n_kv = (int64_t)a->n_past + a->n_tokens;
  if (n_kv > mi::kExactMaxKeys)
    return fail(MI_HIP_E_UNSUPPORTED, "reference-order attention covers up to %d keys", mi::kExactMaxKeys);
  // a KV head's V rows are addressed with 32-bit byte offsets
  if (n_kv * r.v_s2 + 4LL * r.head_dim > INT32_MAX)
    return fail(MI_HIP_E_UNSUPPORTED, "n_kv * position stride exceeds 2^31 bytes for one KV head");
  if ((rc = bind_device())) return rc;
  mi::ExactAttn ea{};
  ea.q = reinterpret_cast<const char*>(a->q);
  ea.k = r.k;
  ea.v = r.v;
  ea.out = reinterpret_cast<char*>(a->out);
  ea.q_s1 = (int64_t)a->q_nb[1];
  ea.q_s2 = (int64_t)a->q_nb[2];
  ea.k_s1 = r.k_s1;
  ea.k_s2 = r.k_s2;
  ea.v_s1 = r.v_s1;
  ea.v_s2 = r.v_s2;
  ea.o_s1 = (int64_t)a->out_nb[1];
  ea.o_s2 = (int64_t)a->out_nb[2];
  ea.n_head = a->n_head;
  ea.n_rep = a->n_rep;
  ea.n_past = a->n_past;
  ea.n_tokens = a->n_tokens;
  ea.head_dim = r.head_dim;
  ea.scale = a->scale;
  const hipError_t e = mi::launch_attn_exact(ea, static_cast<hipStream_t>(a->stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "reference-order attention launch");
}

int mi_hip_attn_decode_batch(const mi_hip_attn_args* items, int n_items, void* stream) {
  if (!items || n_items <= 0) return fail(MI_HIP_E_INVALID, "need at least one item");
  Resolved r0;
  int rc = resolve_kv(&items[0], &r0);
  if (rc) return rc;
  for (int i = 0; i < n_items; ++i) {
    Resolved r;
    if ((rc = resolve_kv(&items[i], &r))) return rc;
    if ((rc = check_problem(&items[i], r))) return rc;
    if (items[i].n_tokens != 1) return fail(MI_HIP_E_INVALID, "item %d: n_tokens must be 1", i);
    if (r.head_dim != r0.head_dim || r.f16 != r0.f16 || r.n_head_kv != r0.n_head_kv ||
        items[i].n_rep != items[0].n_rep || items[i].scale != items[0].scale)
      return fail(MI_HIP_E_INVALID, "item %d: shape, type or scale differs from item 0", i);
  }
  if ((rc = bind_device())) return rc;
  return run_decode(items, n_items, static_cast<hipStream_t>(stream), workspace_of(&items[0]));
}

int mi_hip_attn_decode_batch_noalloc(const mi_hip_attn_args* items, int n_items, void* stream) {
  if (!items || n_items <= 0) return fail(MI_HIP_E_INVALID, "need at least one item");
  Resolved r0;
  int rc = resolve_kv(&items[0], &r0);
  if (rc) return rc;
  for (int i = 0; i < n_items; ++i) {
    Resolved r;
    if ((rc = resolve_kv(&items[i], &r))) return rc;
    if ((rc = check_problem(&items[i], r))) return rc;
    if (items[i].n_tokens != 1) return fail(MI_HIP_E_INVALID, "item %d: n_tokens must be 1", i);
    if (r.head_dim != r0.head_dim || r.f16 != r0.f16 || r.n_head_kv != r0.n_head_kv ||
        items[i].n_rep != items[0].n_rep || items[i].scale != items[0].scale)
      return fail(MI_HIP_E_INVALID, "item %d: shape, type or scale differs from item 0", i);
  }
  if ((rc = bind_device())) return rc;
  // run_decode refuses launches beyond the scratch's groups or record bytes.
  return run_decode(items, n_items, static_cast<hipStream_t>(stream), g.scratch_ws);
}

int mi_hip_op_attn_qk(mi_tensor* dst, void* stream) {
  if (!dst || dst->op != MI_OP_ATTN_QK) return fail(MI_HIP_E_INVALID, "dst is not an ATTN_QK node");
  const mi_tensor* q = dst->src[0];
  const mi_tensor* k = dst->src[1];
  int rc;
  if ((rc = check_f32(dst, "scores")) || (rc = check_f32(q, "Q")) || (rc = check_kv_tensor(k, "K")))
    return rc;
  const int n_rep = mi_tensor_param_i32(dst, 1);
  if (n_rep <= 0) return fail(MI_HIP_E_INVALID, "n_rep must be positive");
  if (dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || k->ne[0] != q->ne[0])
    return fail(MI_HIP_E_INVALID, "ATTN_QK shapes are inconsistent");
  if ((q->ne[1] - 1) / n_rep >= k->ne[1] || dst->ne[0] > k->ne[2])
    return fail(MI_HIP_E_INVALID, "ATTN_QK reads outside the K tensor");
  if ((rc = bind_device())) return rc;
  hipError_t e = mi::launch_attn_qk_node(view_of(dst), view_of(q), view_of(k),
                                         k->type == MI_TYPE_F16, n_rep,
                                         static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "attn_qk launch");
}

int mi_hip_op_softmax(mi_tensor* dst, void* stream) {
  if (!dst || dst->op != MI_OP_SOFTMAX) return fail(MI_HIP_E_INVALID, "dst is not a SOFTMAX node");
  const mi_tensor* s = dst->src[0];
  int rc;
  if ((rc = check_f32(dst, "probs")) || (rc = check_f32(s, "scores"))) return rc;
  for (int i = 0; i < 3; ++i)
    if (dst->ne[i] != s->ne[i]) return fail(MI_HIP_E_INVALID, "SOFTMAX shape differs from its source");
  const int n_past = mi_tensor_param_i32(dst, 0);
  if (n_past < 0) return fail(MI_HIP_E_INVALID, "n_past must be >= 0");
  if ((rc = bind_device())) return rc;
  hipError_t e = mi::launch_softmax_node(view_of(dst), view_of(s), n_past,
                                         mi_tensor_param_f32(dst, 1), static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "softmax launch");
}

namespace {

// freq[p] = base^(-2p / n_dims) for p < n_dims / 2, each a float powf exactly
// as src/ops_cpu.cpp:289 evaluates it (the device then forms pos * freq[p]
// with one rounded product, as the engine does).
void rope_freqs(float* freq, int n_dims, float base) {
  for (int p = 0; p < n_dims / 2; ++p) freq[p] = std::pow(base, -(float)(2 * p) / (float)n_dims);
}

int check_rope_dims(int n_dims, int head_dim) {
  if (n_dims < 0 || n_dims % 2 || n_dims > head_dim || n_dims > 2 * mi::kRopeMaxPairs)
    return fail(MI_HIP_E_UNSUPPORTED, "n_dims %d: must be even, in [0, head_dim = %d] and <= %d",
                n_dims, head_dim, 2 * mi::kRopeMaxPairs);
  return MI_HIP_OK;
}

bool strides4(const size_t nb[3]) { return nb[0] % 4 == 0 && nb[1] % 4 == 0 && nb[2] % 4 == 0; }

}  // namespace

int mi_hip_op_rope(mi_tensor* dst, void* stream) {
  if (!dst || dst->op != MI_OP_ROPE) return fail(MI_HIP_E_INVALID, "dst is not a ROPE node");
  const mi_tensor* s = dst->src[0];
  int rc;
  if ((rc = check_f32(dst, "dst")) || (rc = check_f32(s, "src"))) return rc;
  for (int i = 0; i < 3; ++i)
    if (dst->ne[i] != s->ne[i]) return fail(MI_HIP_E_INVALID, "ROPE shape differs from its source");
  if (!strides4(dst->nb) || !strides4(s->nb))
    return fail(MI_HIP_E_INVALID, "ROPE strides must be multiples of 4 bytes");
  const int n_past = mi_tensor_param_i32(dst, 0), n_dims = mi_tensor_param_i32(dst, 1);
  if (s->ne[0] > INT32_MAX || s->ne[1] > INT32_MAX || s->ne[2] > INT32_MAX)
    return fail(MI_HIP_E_UNSUPPORTED, "ROPE extents beyond 2^31");
  if ((rc = check_rope_dims(n_dims, (int)s->ne[0]))) return rc;
  if (n_past < 0 || (int64_t)n_past + s->ne[2] > INT32_MAX)
    return fail(MI_HIP_E_INVALID, "positions n_past + token must lie in [0, 2^31)");
  mi::RopeNode p{};
  p.src = static_cast<const char*>(s->data);
  p.dst = static_cast<char*>(dst->data);
  for (int i = 0; i < 3; ++i) {
    p.src_nb[i] = (int64_t)s->nb[i];
    p.dst_nb[i] = (int64_t)dst->nb[i];
  }
  p.rows = s->ne[1] * s->ne[2];
  p.n_heads = (int32_t)s->ne[1];
  p.head_dim = (int32_t)s->ne[0];
  p.n_past = n_past;
  p.n_dims = n_dims;
  rope_freqs(p.freq, n_dims, mi_tensor_param_f32(dst, 2));
  if ((rc = bind_device())) return rc;
  hipError_t e = mi::launch_rope_node(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "rope launch");
}

int mi_hip_rope_append(const mi_hip_rope_args* a) {
  if (!a || !a->kv || !a->k || !a->v) return fail(MI_HIP_E_INVALID, "args, kv, k and v must be non-NULL");
  const mi_hip_kv* kv = a->kv;
  if (a->layer < 0 || a->layer >= kv->d.n_layer)
    return fail(MI_HIP_E_INVALID, "layer %d out of range [0, %d)", a->layer, kv->d.n_layer);
  if (a->n_past < 0 || a->n_tokens < 0 || (int64_t)a->n_past + a->n_tokens > kv->d.n_ctx)
    return fail(MI_HIP_E_INVALID, "positions [%d, %d) outside [0, %d)", a->n_past,
                a->n_past + a->n_tokens, kv->d.n_ctx);
  int rc;
  if ((rc = check_rope_dims(a->n_dims, kv->d.head_dim))) return rc;
  if (a->q) {
    if (!a->q_out) return fail(MI_HIP_E_INVALID, "q_out is NULL");
    if (a->n_head <= 0 || a->n_head % kv->d.n_head_kv)
      return fail(MI_HIP_E_INVALID, "n_head %d must be a positive multiple of n_head_kv %d",
                  a->n_head, kv->d.n_head_kv);
    if (!strides4(a->q_nb) || !strides4(a->q_out_nb))
      return fail(MI_HIP_E_INVALID, "Q strides must be multiples of 4 bytes");
  }
  if (!strides4(a->k_nb) || !strides4(a->v_nb))
    return fail(MI_HIP_E_INVALID, "K/V strides must be multiples of 4 bytes");
  if (a->n_tokens == 0) return MI_HIP_OK;
  mi::RopeAppend p{};
  p.q = reinterpret_cast<const char*>(a->q);
  p.q_out = reinterpret_cast<char*>(a->q_out);
  p.k = reinterpret_cast<const char*>(a->k);
  p.v = reinterpret_cast<const char*>(a->v);
  p.k_cache = kv->tensor(a->layer, 0);
  p.v_cache = kv->tensor(a->layer, 1);
  for (int i = 0; i < 3; ++i) {
    p.q_nb[i] = (int64_t)a->q_nb[i];
    p.qo_nb[i] = (int64_t)a->q_out_nb[i];
    p.k_nb[i] = (int64_t)a->k_nb[i];
    p.v_nb[i] = (int64_t)a->v_nb[i];
  }
  p.c_s1 = kv->s1;
  p.c_s2 = kv->s2;
  p.n_tokens = a->n_tokens;
  p.n_head = a->q ? a->n_head : 0;
  p.n_head_kv = kv->d.n_head_kv;
  p.head_dim = kv->d.head_dim;
  p.n_past = a->n_past;
  p.n_dims = a->n_dims;
  rope_freqs(p.freq, a->n_dims, a->freq_base);
  if ((rc = bind_device())) return rc;
  hipError_t e = mi::launch_rope_append(p, kv->elt == 2, static_cast<hipStream_t>(a->stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "rope append launch");
}

int mi_hip_op_quantize_q8_0(mi_tensor* dst, void* stream) {
  if (!dst || dst->op != MI_OP_QUANTIZE_Q8_0)
    return fail(MI_HIP_E_INVALID, "dst is not a QUANTIZE_Q8_0 node");
  const mi_tensor* s = dst->src[0];
  int rc;
  if ((rc = check_f32(s, "src"))) return rc;
  if (!dst->data) return fail(MI_HIP_E_INVALID, "dst: missing data");
  if (dst->type != MI_TYPE_Q8_0_ACT) return fail(MI_HIP_E_UNSUPPORTED, "dst must be Q8_0_ACT");
  for (int i = 0; i < 4; ++i)
    if (dst->ne[i] != s->ne[i]) return fail(MI_HIP_E_INVALID, "QUANTIZE_Q8_0 shape differs from its source");
  if (s->ne[0] % 32) return fail(MI_HIP_E_INVALID, "ne[0] = %lld is not a multiple of 32", (long long)s->ne[0]);
  if (s->nb[0] != 4) return fail(MI_HIP_E_UNSUPPORTED, "src rows must be contiguous (nb[0] = 4)");
  for (int i = 1; i < 4; ++i)
    if (s->nb[i] % 4 || dst->nb[i] % 4)
      return fail(MI_HIP_E_INVALID, "QUANTIZE_Q8_0 strides must be multiples of 4 bytes");
  mi::Q8Quantize p{};
  p.src = static_cast<const char*>(s->data);
  p.dst = static_cast<char*>(dst->data);
  for (int i = 0; i < 4; ++i) {
    p.src_nb[i] = (int64_t)s->nb[i];
    p.dst_nb[i] = (int64_t)dst->nb[i];
  }
  p.ne0 = s->ne[0];
  p.ne1 = s->ne[1];
  p.ne2 = s->ne[2];
  p.rows = s->ne[1] * s->ne[2] * s->ne[3];
  if ((rc = bind_device())) return rc;
  hipError_t e = mi::launch_quantize_q8_0_act(p, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "quantize launch");
}

int mi_hip_op_mul_mat(mi_tensor* dst, void* stream) {
  if (!dst || dst->op != MI_OP_MUL_MAT) return fail(MI_HIP_E_INVALID, "dst is not a MUL_MAT node");
  const mi_tensor* a = dst->src[0];
  const mi_tensor* b = dst->src[1];
  int rc;
  if ((rc = check_f32(dst, "dst"))) return rc;
  if (!a || !a->data || !b || !b->data) return fail(MI_HIP_E_INVALID, "MUL_MAT: missing operand");
  if (a->type != MI_TYPE_Q8_0) return fail(MI_HIP_E_UNSUPPORTED, "MUL_MAT: only Q8_0 weights (type %d)", (int)a->type);
  if (b->type != MI_TYPE_Q8_0_ACT)
    return fail(MI_HIP_E_INVALID, "MUL_MAT: src[1] must be the Q8_0_ACT output of QUANTIZE_Q8_0");
  const int64_t k = a->ne[0], n = a->ne[1], m = b->ne[1];
  if (k % 32 || b->ne[0] != k) return fail(MI_HIP_E_INVALID, "MUL_MAT: k = %lld must match and be a multiple of 32", (long long)k);
  if (dst->ne[0] != n || dst->ne[1] != m || a->ne[2] * a->ne[3] != 1 || b->ne[2] * b->ne[3] != 1)
    return fail(MI_HIP_E_INVALID, "MUL_MAT shapes are inconsistent");
  if (a->nb[1] % 2 || a->nb[1] < (size_t)(k / 32 * 34) || b->nb[1] % 4 || b->nb[1] < (size_t)(k / 32 * 36) ||
      dst->nb[0] % 4 || dst->nb[1] % 4)
    return fail(MI_HIP_E_INVALID, "MUL_MAT strides do not fit the block layouts");
  mi::Q8MulMat p{};
  p.w = static_cast<const char*>(a->data);
  p.a = static_cast<const char*>(b->data);
  p.dst = static_cast<char*>(dst->data);
  p.w_nb1 = (int64_t)a->nb[1];
  p.a_nb1 = (int64_t)b->nb[1];
  p.dst_nb0 = (int64_t)dst->nb[0];
  p.dst_nb1 = (int64_t)dst->nb[1];
  p.k = k;
  p.n = n;
  p.m = m;
  if ((rc = bind_device())) return rc;
  hipError_t e = mi::launch_mul_mat_q8_0(p, g.n_cu, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "mul_mat launch");
}

int mi_hip_op_attn_kqv(mi_tensor* dst, void* stream) {
  if (!dst || dst->op != MI_OP_ATTN_KQV) return fail(MI_HIP_E_INVALID, "dst is not an ATTN_KQV node");
  const mi_tensor* pr = dst->src[0];
  const mi_tensor* v = dst->src[1];
  int rc;
  if ((rc = check_f32(dst, "out")) || (rc = check_f32(pr, "probs")) || (rc = check_kv_tensor(v, "V")))
    return rc;
  const int n_rep = mi_tensor_param_i32(dst, 0);
  if (n_rep <= 0) return fail(MI_HIP_E_INVALID, "n_rep must be positive");
  if (dst->ne[0] != v->ne[0] || dst->ne[1] != pr->ne[2] || dst->ne[2] != pr->ne[1])
    return fail(MI_HIP_E_INVALID, "ATTN_KQV shapes are inconsistent");
  if ((pr->ne[2] - 1) / n_rep >= v->ne[1] || pr->ne[0] > v->ne[2])
    return fail(MI_HIP_E_INVALID, "ATTN_KQV reads outside the V tensor");
  if ((rc = bind_device())) return rc;
  hipError_t e = mi::launch_attn_kqv_node(view_of(dst), view_of(pr), view_of(v),
                                          v->type == MI_TYPE_F16, n_rep,
                                          static_cast<hipStream_t>(stream));
  return e == hipSuccess ? MI_HIP_OK : hip_fail(e, "attn_kqv launch");
}

int mi_hip_op_attn_fused(mi_tensor* dst, void* stream) {
  mi_hip_attn_args a;
  int rc = fused_args_from_nodes(dst, &a);
  if (rc) return rc;
  a.stream = stream;
  return mi_hip_attn_fwd(&a);
}

int mi_hip_graph_prepare(const mi_cgraph* graph) {
  if (!graph || (graph->n_nodes > 0 && !graph->nodes))
    return fail(MI_HIP_E_INVALID, "graph is NULL or has no node array");
  std::lock_guard<std::mutex> lk(g_plan_mu);
  g_readers.clear();
  g_roles.clear();
  for (int i = 0; i < graph->n_nodes; ++i) {
    const mi_tensor* n = graph->nodes[i];
    for (int s = 0; s < MI_MAX_SRC; ++s) {
      const mi_tensor* src = n->src[s];
      if (src && (src->op == MI_OP_ATTN_QK || src->op == MI_OP_SOFTMAX)) {
        int32_t* c = g_readers.find(src, true);
        if (!c) return fail(MI_HIP_E_UNSUPPORTED, "graph too large for the planner");
        ++*c;
      }
    }
  }
  for (int i = 0; i < graph->n_nodes; ++i) {
    const mi_tensor* kqv = graph->nodes[i];
    if (kqv->op != MI_OP_ATTN_KQV) continue;
    const mi_tensor* sm = kqv->src[0];
    if (!sm || sm->op != MI_OP_SOFTMAX) continue;
    const mi_tensor* qk = sm->src[0];
    if (!qk || qk->op != MI_OP_ATTN_QK) continue;
    int32_t* rs = g_readers.find(sm, false);
    int32_t* rq = g_readers.find(qk, false);
    if (!rs || !rq || *rs != 1 || *rq != 1) continue;
    const Binding* bk = find_binding(qk->src[1]);
    const Binding* bv = find_binding(kqv->src[1]);
    if (!bk || !bv || bk->kv != bv->kv || bk->layer != bv->layer || bk->which != 0 || bv->which != 1)
      continue;
    int32_t* a = g_roles.find(qk, true);
    int32_t* b = g_roles.find(sm, true);
    int32_t* c = g_roles.find(kqv, true);
    if (!a || !b || !c) return fail(MI_HIP_E_UNSUPPORTED, "graph too large for the planner");
    *a = kFusedQK;
    *b = kFusedSoftmax;
    *c = kFusedKQV;
  }
  return MI_HIP_OK;
}

namespace {

// Bytes spanned by a tensor's elements from its data pointer.
size_t tensor_extent(const mi_tensor* t) {
  size_t e = t->type == MI_TYPE_F16 ? 2 : 4;
  for (int i = 0; i < 4; ++i)
    if (t->ne[i] > 1) e += (size_t)(t->ne[i] - 1) * t->nb[i];
  return e;
}

// An ATTN_QK, SOFTMAX or ATTN_KQV node whose tensors live in host memory, run
// on the node kernels: its sources are copied into the staging buffer, the
// node runs on device copies of the three tensor headers, and the output is
// copied back before returning (the caller's barrier then publishes it).
int run_host_node(mi_tensor* dst) {
  const int n_src = dst->op == MI_OP_SOFTMAX ? 1 : 2;
  for (int i = 0; i < n_src; ++i)
    if (!dst->src[i] || !dst->src[i]->data) return fail(MI_HIP_E_INVALID, "node source %d has no data", i);
  if (!dst->data) return fail(MI_HIP_E_INVALID, "node output has no data");
  size_t off[3], ext[3], total = 0;
  const mi_tensor* ts[3] = {dst, dst->src[0], n_src > 1 ? dst->src[1] : nullptr};
  for (int i = 0; i < 1 + n_src; ++i) {
    ext[i] = tensor_extent(ts[i]);
    off[i] = total;
    total += (ext[i] + 255) & ~size_t(255);
  }
  int rc;
  if ((rc = bind_device())) return rc;
  std::lock_guard<std::mutex> lk(g.node_mu);
  if (!g.node_stream) MI_TRY_HIP(hipStreamCreateWithFlags(&g.node_stream, hipStreamNonBlocking), "node stream");
  if (total > g.node_stage_bytes) {
    dev_free(g.node_stage, g.node_stage_bytes);
    g.node_stage = nullptr;
    g.node_stage_bytes = 0;
    void* p = nullptr;
    if ((rc = dev_alloc(&p, total, "host-node staging"))) return rc;
    g.node_stage = static_cast<char*>(p);
    g.node_stage_bytes = total;
  }
  mi_tensor dev[3];
  for (int i = 0; i < 1 + n_src; ++i) {
    dev[i] = *ts[i];
    dev[i].data = g.node_stage + off[i];
    if (i > 0)
      MI_TRY_HIP(hipMemcpyAsync(dev[i].data, ts[i]->data, ext[i], hipMemcpyHostToDevice, g.node_stream),
                 "node source copy");
  }
  dev[0].src[0] = &dev[1];
  dev[0].src[1] = n_src > 1 ? &dev[2] : nullptr;
  void* st = g.node_stream;
  rc = dst->op == MI_OP_ATTN_QK ? mi_hip_op_attn_qk(&dev[0], st)
       : dst->op == MI_OP_SOFTMAX ? mi_hip_op_softmax(&dev[0], st)
                                  : mi_hip_op_attn_kqv(&dev[0], st);
  if (rc) return rc;
  MI_TRY_HIP(hipMemcpyAsync(dst->data, dev[0].data, ext[0], hipMemcpyDeviceToHost, g.node_stream), "node output copy");
  MI_TRY_HIP(hipStreamSynchronize(g.node_stream), "node stream sync");
  return MI_HIP_OK;
}

}  // namespace

int mi_hip_set_host_nodes(int32_t on) {
  if (on != 0 && on != 1) return fail(MI_HIP_E_INVALID, "on must be 0 or 1");
  g.host_nodes.store(on);
  return MI_HIP_OK;
}

int mi_hip_compute_forward(mi_tensor* dst, int ith, int nth) {
  (void)nth;
  if (!dst) return 0;
  switch (dst->op) {
    case MI_OP_CPY: {
      const mi_tensor* owner = dst->view_src ? dst->view_src : dst;
      const Binding* b = find_binding(owner);
      if (!b) return 0;
      if (ith != 0) return 1;
      mi_hip_kv* kv = b->kv;
      const mi_tensor* src = dst->src[0];
      if (!src || src->type != MI_TYPE_F32 || !src->data) {
        fail(MI_HIP_E_INVALID, "CPY into the KV cache needs an F32 host source");
        return -1;
      }
      if (dst->nb[2] != owner->nb[2] || dst->view_offs % owner->nb[2] != 0) {
        fail(MI_HIP_E_INVALID, "CPY destination is not a whole-position view of the cache");
        return -1;
      }
      if (src->ne[0] != kv->d.head_dim || src->ne[1] != kv->d.n_head_kv || src->ne[2] != dst->ne[2]) {
        fail(MI_HIP_E_INVALID, "CPY source shape does not match the cache rows");
        return -1;
      }
      const int pos0 = (int)(dst->view_offs / owner->nb[2]);
      return mi_hip_kv_write(kv, b->layer, b->which, pos0, (int)dst->ne[2],
                             static_cast<const float*>(src->data), src->nb, 0, kv->stream) == MI_HIP_OK
                 ? 1
                 : -1;
    }
    case MI_OP_ATTN_QK:
    case MI_OP_SOFTMAX:
    case MI_OP_ATTN_KQV: {
      const int32_t role = role_of(dst);
      if (role == kFusedQK || role == kFusedSoftmax) return 1;
      if (role != kFusedKQV) {
        const mi_tensor* kvsrc = dst->op == MI_OP_SOFTMAX ? nullptr : dst->src[1];
        if (kvsrc && find_binding(kvsrc)) {
          fail(MI_HIP_E_STATE,
               "attention node reads a device-resident KV cache but is not part of a planned fused "
               "chain (call mi_hip_graph_prepare after allocation)");
          return -1;
        }
        if (!g.host_nodes.load()) return 0;
        if (ith != 0) return 1;
        return run_host_node(dst) == MI_HIP_OK ? 1 : -1;
      }
      if (ith != 0) return 1;
      const mi_tensor* sm = dst->src[0];
      const mi_tensor* qk = sm->src[0];
      const mi_tensor* q = qk->src[0];
      const Binding* b = find_binding(qk->src[1]);
      if (!b) {
        fail(MI_HIP_E_STATE, "K tensor lost its binding");
        return -1;
      }
      mi_hip_kv* kv = b->kv;
      if (q->type != MI_TYPE_F32 || !contiguous3(q) || dst->type != MI_TYPE_F32 || !contiguous3(dst)) {
        fail(MI_HIP_E_UNSUPPORTED, "host Q and output must be contiguous F32");
        return -1;
      }
      const size_t n = (size_t)q->ne[0] * q->ne[1] * q->ne[2];
      if (n > kv->q_floats || q->ne[0] != kv->d.head_dim) {
        fail(MI_HIP_E_INVALID, "Q does not fit the cache's staging (n_ctx x n_head x head_dim)");
        return -1;
      }
      if (bind_device()) return -1;
      float* sq = kv->stage;
      float* so = kv->stage + kv->q_floats;
      mi_hip_attn_args a;
      std::memset(&a, 0, sizeof a);
      a.kv = kv;
      a.layer = b->layer;
      a.q = sq;
      a.out = so;
      a.q_nb[0] = a.out_nb[0] = 4;
      a.q_nb[1] = a.out_nb[1] = 4 * (size_t)q->ne[0];
      a.q_nb[2] = a.out_nb[2] = 4 * (size_t)q->ne[0] * q->ne[1];
      a.n_head = (int32_t)q->ne[1];
      a.n_rep = mi_tensor_param_i32(qk, 1);
      a.n_past = mi_tensor_param_i32(qk, 0);
      a.n_tokens = (int32_t)q->ne[2];
      a.scale = mi_tensor_param_f32(sm, 1);
      a.stream = kv->stream;
      if (qk->ne[0] != (int64_t)a.n_past + a.n_tokens || mi_tensor_param_i32(sm, 0) != a.n_past) {
        fail(MI_HIP_E_INVALID, "fused chain op_params disagree with the shapes");
        return -1;
      }
      hipError_t e = hipMemcpyAsync(sq, q->data, n * sizeof(float), hipMemcpyHostToDevice, kv->stream);
      if (e != hipSuccess) {
        hip_fail(e, "hipMemcpyAsync(Q)");
        return -1;
      }
      if (mi_hip_attn_fwd(&a) != MI_HIP_OK) return -1;
      e = hipMemcpyAsync(dst->data, so, n * sizeof(float), hipMemcpyDeviceToHost, kv->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(kv->stream);
      if (e != hipSuccess) {
        hip_fail(e, "attention output copy");
        return -1;
      }
      return 1;
    }
    default:
      return 0;
  }
}

}  // extern "C"
