"""Benchmark of the fused GQA attention kernels on one MI355X.

Headline (one "step" = one pass of the hot path over one batch):
  decode attention, 24 layers' independent caches at n_kv = 4096, Qwen2.5-0.5B
  heads (14 Q / 2 KV, head_dim 64), F32 cache, one batched launch. `value` is
  the algorithmic HBM bytes (K + V + Q + O) per step / time per step. Steps
  rotate over several cache sets (> 256 MB in total) so reads come from HBM,
  not the 256 MB Infinity Cache.
Also reported (secondary, same run): prefill-1024 and -4096 causal attention
TFLOP/s (causal FLOPs 4*D*H*n(n+1)/2), the Qwen2.5-7B-shape F16-cache decode
at n_kv = 8192, the engine's per-layer call pattern (24 single launches), the
Q8_0 output-projection matvec, and end-to-end greedy generation on the device
engine (tokens/s, attention time per token, ids against the reference engine,
the reference CPU engine's own --bench on the host cores beside it).
The CPU baseline times the reference's three-node path (attn_qk -> softmax ->
attn_kqv with a barrier per node) on the host cores on a bounded sample.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "mini-infer-llama.cpp_amd")
sys.path.insert(0, ROOT)
sys.path.insert(0, PKG)

METRIC = "decode attn GB/s (% HBM peak) @ n_kv=4096; prefill-1024 attn TFLOP/s"
HBM_PEAK_GBPS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--nondeterministic", action="store_true",
                    help="waves take work from a counter in the fused kernels (mi_hip_set_deterministic(0))")
    ap.add_argument("--only", default="",
                    help="comma list: decode,streams,sweep,prefill,d7b,perlayer,q8,memread,e2e,copy (copy: the "
                         "counter calibration workload, only when named)")
    return ap.parse_args()


def decode_bytes(n_layers, n_kv, h, hkv, d, kv_elt):
    return n_layers * (2 * n_kv * hkv * d * kv_elt + 2 * h * d * 4)


def causal_flops(n, h, d):
    return 4 * d * h * n * (n + 1) // 2


SPINUP_S = 0.03


def spin_up(torch, launch, seconds=SPINUP_S):
    """Untimed launches of the same step for `seconds` of wall time before a
    measurement: the GPU's clock ramps over the first ~15-20 ms of continuous
    work after an idle gap (measured: prefill-1024 blocks of 220 launches ran
    26.8, 25.7, 24.8, then 24.3 us per launch steadily), and every measurement
    here follows host-side setup that leaves the device idle."""
    t0 = time.perf_counter()
    i = 0
    while True:
        for _ in range(64):
            launch(i)
            i += 1
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def run_timed(torch, launch, steps, warmup):
    """A clock spin-up (spin_up), warmup untimed steps, then `steps` timed steps
    back to back, bracketed by synchronize and by two HIP events on the stream
    the kernels run on; returns ms per step. (Events between the launches would
    put their own commands between the kernels, so the per-launch time of a
    one-launch step is this same figure; rocprofv3 gives the kernel's own
    duration.)"""
    spin_up(torch, launch)
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        launch(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def bench_decode(torch, mh, lib, stream, steps, warmup, n_layers=24, n_kv=4096, h=14, hkv=2,
                 d=64, f16=False, sets=None):
    elt = 2 if f16 else 4
    per_set = n_layers * 2 * n_kv * hkv * d * elt
    if sets is None:
        sets = max(3, -(-600 * 2**20 // per_set))  # > 256 MB MALL, about 600 MB rotated
    gen = torch.Generator(device="cuda").manual_seed(4096)
    dt = torch.float16 if f16 else torch.float32
    arrays = []
    for s in range(sets):
        k = torch.randn((n_layers, n_kv, hkv, d), device="cuda", generator=gen).to(dt)
        v = torch.randn((n_layers, n_kv, hkv, d), device="cuda", generator=gen).to(dt)
        q = torch.randn((n_layers, 1, h, d), device="cuda", generator=gen)
        o = torch.empty((n_layers, 1, h, d), device="cuda")
        items = (mh.AttnArgs * n_layers)(*[
            mh.attn_args(q[l], o[l], h // hkv, n_kv - 1, float(d) ** -0.5, stream, k=k[l], v=v[l])
            for l in range(n_layers)])
        arrays.append((k, v, q, o, items))

    def launch(i):
        items = arrays[i % sets][4]
        rc = lib.mi_hip_attn_decode_batch(items, n_layers, stream)
        if rc:
            raise mh.MiHipError(rc, lib.last_error())

    ms = run_timed(torch, launch, steps, warmup)
    kern_ms = ms  # one launch per step
    nbytes = decode_bytes(n_layers, n_kv, h, hkv, d, elt)
    return dict(ms_per_step=ms, kernel_ms=kern_ms, bytes=nbytes, sets=sets,
                gbps=nbytes / (ms * 1e-3) / 1e9, kernel_gbps=nbytes / (kern_ms * 1e-3) / 1e9)


def bench_decode_streams(torch, mh, lib, steps, warmup, n_streams=2, n_layers=24, n_kv=4096, h=14, hkv=2,
                         d=64):
    """The headline decode with independent batches alternating over n_streams
    streams, each stream with its own decode workspace (so launches on
    different streams may overlap): per-launch throughput when one launch's
    start overlaps another's tail. The same kernels and work per launch; a
    launch's workgroups are then not all resident at once, which the early
    merge's bounded wait covers (its fallbacks are counted and reported)."""
    sets = 2 * n_streams
    gen = torch.Generator(device="cuda").manual_seed(4097)
    streams = [torch.cuda.Stream() for _ in range(n_streams)]  # default priority
    wss = [lib.workspace_create(hkv, h, d) for _ in range(n_streams)]
    arrays = []
    for s in range(sets):
        st = streams[s % n_streams]
        k = torch.randn((n_layers, n_kv, hkv, d), device="cuda", generator=gen)
        v = torch.randn((n_layers, n_kv, hkv, d), device="cuda", generator=gen)
        q = torch.randn((n_layers, 1, h, d), device="cuda", generator=gen)
        o = torch.empty((n_layers, 1, h, d), device="cuda")
        items = (mh.AttnArgs * n_layers)(*[
            mh.attn_args(q[l], o[l], h // hkv, n_kv - 1, float(d) ** -0.5, st.cuda_stream, k=k[l], v=v[l],
                         ws=wss[s % n_streams])
            for l in range(n_layers)])
        arrays.append((k, v, q, o, items))
    torch.cuda.synchronize()

    def launch(i):
        rc = lib.mi_hip_attn_decode_batch(arrays[i % sets][4], n_layers, streams[i % n_streams].cuda_stream)
        if rc:
            raise mh.MiHipError(rc, lib.last_error())

    try:
        for i in range(warmup):
            launch(i)
        torch.cuda.synchronize()
        for ws in wss:
            lib.workspace_check(ws, streams[0].cuda_stream)
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(streams[0])
        for st in streams[1:]:
            st.wait_event(t0)
        for i in range(steps):
            launch(i)
        for st in streams[1:]:
            ev = torch.cuda.Event()
            ev.record(st)
            streams[0].wait_event(ev)
        t1.record(streams[0])
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        fallbacks = lost = 0
        for ws in wss:
            rc, fb, lo = lib.workspace_check(ws, streams[0].cuda_stream)
            fallbacks += fb
            lost += lo
    finally:
        torch.cuda.synchronize()
        for ws in wss:
            lib.check(lib.mi_hip_workspace_destroy(ws))
    nbytes = decode_bytes(n_layers, n_kv, h, hkv, d, 4)
    return dict(streams=n_streams, us_per_launch=ms * 1e3, gbps=nbytes / (ms * 1e-3) / 1e9,
                early_fallbacks=fallbacks, lost_groups=lost)


def bench_decode_per_layer(torch, mh, lib, stream, steps, warmup, n_layers=24, n_kv=4096):
    """The engine's call pattern: one fused launch per layer node."""
    h, hkv, d = 14, 2, 64
    sets = 6
    gen = torch.Generator(device="cuda").manual_seed(99)
    per = []
    for s in range(sets):
        k = torch.randn((n_layers, n_kv, hkv, d), device="cuda", generator=gen)
        v = torch.randn((n_layers, n_kv, hkv, d), device="cuda", generator=gen)
        q = torch.randn((n_layers, 1, h, d), device="cuda", generator=gen)
        o = torch.empty((n_layers, 1, h, d), device="cuda")
        args = [mh.attn_args(q[l], o[l], 7, n_kv - 1, 0.125, stream, k=k[l], v=v[l])
                for l in range(n_layers)]
        per.append((k, v, q, o, args))

    def launch(i):
        for a in per[i % sets][4]:
            rc = lib.mi_hip_attn_fwd(ctypes.byref(a))
            if rc:
                raise mh.MiHipError(rc, lib.last_error())

    ms = run_timed(torch, launch, max(5, steps // 4), max(2, warmup // 4))
    nbytes = decode_bytes(n_layers, n_kv, h, hkv, d, 4)
    return dict(us_per_layer=ms * 1e3 / n_layers, gbps=nbytes / (ms * 1e-3) / 1e9)


def bench_prefill(torch, mh, lib, stream, steps, warmup, n, h=14, hkv=2, d=64, f16=False):
    gen = torch.Generator(device="cuda").manual_seed(n)
    dt = torch.float16 if f16 else torch.float32
    q = torch.randn((n, h, d), device="cuda", generator=gen)
    k = torch.randn((n, hkv, d), device="cuda", generator=gen).to(dt)
    v = torch.randn((n, hkv, d), device="cuda", generator=gen).to(dt)
    o = torch.empty((n, h, d), device="cuda")
    a = mh.attn_args(q, o, h // hkv, 0, float(d) ** -0.5, stream, k=k, v=v)

    def launch(i):
        rc = lib.mi_hip_attn_fwd(ctypes.byref(a))
        if rc:
            raise mh.MiHipError(rc, lib.last_error())

    ms = run_timed(torch, launch, steps, warmup)
    kern_ms = ms  # one launch per step
    flops = causal_flops(n, h, d)
    return dict(n=n, ms_per_step=ms, kernel_ms=kern_ms, flops=flops,
                tflops=flops / (kern_ms * 1e-3) / 1e12)


def q8_weight_tensor(torch, gen, n, k):
    """Random Q8_0 weight rows on the device: fp16 scales in [1e-4, 4e-3), int8
    values in [-127, 127], packed as the 34-byte GGUF blocks."""
    nb = k // 32
    blocks = torch.empty((n, nb, 34), dtype=torch.uint8, device="cuda")
    scale = (torch.rand((n, nb), device="cuda", generator=gen) * 4e-3 + 1e-4).to(torch.float16)
    blocks[:, :, :2] = scale.view(torch.uint8).view(n, nb, 2)
    blocks[:, :, 2:] = torch.randint(-127, 128, (n, nb, 32), device="cuda", generator=gen,
                                     dtype=torch.int8).view(torch.uint8)
    return blocks.view(n, nb * 34)


def bench_q8_matvec(torch, mh, lib, stream, steps, warmup, n=151936, k=896, sets=3):
    """MUL_MAT with Q8_0 weights for one token: the output projection of
    Qwen2.5-0.5B (151936 x 896, tied to the token embedding), the largest
    matrix-vector product of a decode step; weight sets rotated beyond the
    256 MB MALL. One QUANTIZE_Q8_0 of the activation, then timed MUL_MATs."""
    gen = torch.Generator(device="cuda").manual_seed(151936)
    ws = [q8_weight_tensor(torch, gen, n, k) for _ in range(sets)]
    x = torch.randn((1, k), device="cuda", generator=gen)
    act = torch.empty((k // 32 * 36,), dtype=torch.uint8, device="cuda")
    out = torch.empty((1, n), device="cuda")
    xt = mh.make_tensor(x.data_ptr(), [k, 1], [4, 4 * k])
    qn = mh.make_tensor(act.data_ptr(), [k, 1], [36, k // 32 * 36], type_=mh.MI_TYPE_Q8_0_ACT,
                        op=mh.MI_OP_QUANTIZE_Q8_0, src=[xt])
    lib.check(lib.mi_hip_op_quantize_q8_0(ctypes.byref(qn), stream))
    nodes = []
    for w in ws:
        wt = mh.make_tensor(w.data_ptr(), [k, n], [34, k // 32 * 34], type_=mh.MI_TYPE_Q8_0)
        nodes.append((wt, mh.make_tensor(out.data_ptr(), [n, 1], [4, 4 * n],
                                         op=mh.MI_OP_MUL_MAT, src=[wt, qn])))

    def launch(i):
        rc = lib.mi_hip_op_mul_mat(ctypes.byref(nodes[i % sets][1]), stream)
        if rc:
            raise mh.MiHipError(rc, lib.last_error())

    ms = run_timed(torch, launch, steps, warmup)
    nbytes = n * (k // 32 * 34) + k // 32 * 36 + 4 * n
    return dict(n=n, k=k, kernel_ms=ms, bytes=nbytes, gbps=nbytes / (ms * 1e-3) / 1e9, sets=sets)


def bench_copy(torch, steps, warmup, nbytes=256 << 20):
    """A plain device-to-device copy of known size: the calibration workload for
    the FETCH_SIZE / WRITE_SIZE counters (bytes read = bytes written = nbytes)."""
    src = torch.empty(nbytes // 4, device="cuda").uniform_()
    dst = torch.empty_like(src)
    kern_ms = run_timed(torch, lambda i: dst.copy_(src), steps, warmup)
    return dict(bytes=nbytes, kernel_ms=kern_ms, gbps=2 * nbytes / (kern_ms * 1e-3) / 1e9)


def device_info():
    """CU count and peak engine clock of the gfx950 agent as rocminfo reports
    them (None where rocminfo is absent)."""
    info = {"cus": None, "max_clock_mhz": None}
    try:
        txt = subprocess.run(["/opt/rocm/bin/rocminfo"], capture_output=True, text=True,
                             timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        return info
    for agent in txt.split("Agent ")[1:]:
        if "gfx950" not in agent:
            continue
        cu = re.search(r"Compute Unit:\s+(\d+)", agent)
        clk = re.search(r"Max Clock Freq\. \(MHz\):\s+(\d+)", agent)
        info["cus"] = int(cu.group(1)) if cu else None
        info["max_clock_mhz"] = int(clk.group(1)) if clk else None
        break
    return info


def bench_memread(torch, lib, stream, steps, warmup, nbytes=1 << 30,
                  shapes=(1024, 2048, 4096, 8192, 16384)):
    """The measured read-bandwidth ceiling (mi_hip_memread, the device
    counterpart of tools/bench_memread.cpp): a load-and-accumulate pass over
    1 GiB (4x the 256 MB MALL), back to back, at several workgroup counts;
    the fastest is the ceiling."""
    src = torch.empty(nbytes // 4, device="cuda").uniform_()
    sums = torch.empty(max(shapes), device="cuda")
    a, s = ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(sums.data_ptr())
    per = {}
    for n in shapes:
        ms = run_timed(torch, lambda i: lib.check(lib.mi_hip_memread(a, nbytes, s, n, stream)),
                       steps, warmup)
        torch.cuda.synchronize()
        total = float(sums[:n].double().sum().item())
        assert abs(total / (nbytes // 4) - 0.5) < 0.01, "read pass sums disagree with the buffer"
        per[n] = nbytes / (ms * 1e-3) / 1e9
    best = max(per, key=per.get)
    return dict(bytes=nbytes, n_sums=best, gbps=per[best],
                gbps_by_workgroups={str(k): round(v, 1) for k, v in per.items()})


def bench_read_floor(torch, lib, stream, steps, warmup, nbytes, sets=7,
                     shapes=(240, 256, 512, 1024, 2048)):
    """The read floor of the headline step: mi_hip_memread over exactly the
    step's cache bytes (24 layers x n_kv 4096 x 2 KV heads x (K + V) x 64 F32),
    over `sets` buffers rotated as the decode's cache sets are, launched back
    to back; the fastest workgroup count is the floor."""
    bufs = [torch.empty(nbytes // 4, device="cuda").uniform_() for _ in range(sets)]
    sums = torch.empty(max(shapes), device="cuda")
    ptrs = [ctypes.c_void_p(b.data_ptr()) for b in bufs]
    s = ctypes.c_void_p(sums.data_ptr())
    per = {}
    for n in shapes:
        ms = run_timed(torch, lambda i: lib.check(lib.mi_hip_memread(ptrs[i % sets], nbytes, s, n, stream)),
                       steps, warmup)
        per[n] = ms
    best = min(per, key=per.get)
    return dict(bytes=nbytes, sets=sets, workgroups=best, us=per[best] * 1e3,
                gbps=nbytes / (per[best] * 1e-3) / 1e9,
                us_by_workgroups={str(k): round(v * 1e3, 3) for k, v in per.items()})


E2E_SEED = 1234


def bench_e2e(mh):
    """End-to-end greedy generation (the reference CLI's loop, src/main.cpp:474-495)
    on the random-init Qwen2.5-0.5B-shaped Q8_0 model: 128 seeded prompt ids,
    one prefill call, 255 decode calls, n_ctx 2048. Fused attention timed plain
    (tokens/s) and with per-layer attention events (attention time per token);
    the reference-order mode's ids are checked against the reference engine's."""
    import tempfile
    import qwen2_gguf as gg
    from qwen2 import Qwen2, fork_summary, teacher_forced
    d = tempfile.mkdtemp(prefix="mi_e2e_")
    path = os.path.join(d, "qwen05_q8_0.gguf")
    sha = gg.write_qwen2_q8_0(path, E2E_SEED)
    prompt = gg.prompt_ids(E2E_SEED, 128, gg.QWEN2_05B["n_vocab"])
    with open(os.path.join(ROOT, "tests", "golden", "e2e_qwen05_q8_0.json")) as f:
        gold = json.load(f)
    out = {"workload": "Qwen2.5-0.5B-shaped random-init Q8_0 GGUF (seed 1234), 128-token prompt, "
                       "256 greedy ids (1 prefill + 255 decode calls), n_ctx 2048",
           "model_sha256_ok": sha == gold["model_sha256"]}
    free = {}
    with Qwen2(path, n_ctx=2048, max_tokens=len(prompt)) as m:
        for mode, key in ((mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER, "reference_order"),
                          (mh.MI_HIP_QWEN2_ATTN_FUSED, "fused")):
            m.set_attention(mode)
            m.generate(prompt[:8], 4)  # warm-up
            t0 = time.perf_counter()
            nxt, _ = m.forward(prompt, n_past=0)
            t1 = time.perf_counter()
            ids = [nxt]
            for i in range(255):
                nxt, _ = m.forward([nxt], n_past=len(prompt) + i)
                ids.append(nxt)
            t2 = time.perf_counter()
            # the same loop with every step on the device (no host round trip
            # between steps): decode rate from a 256-id run less a 1-id run
            dl = []
            for n_pred in (1, 256, 1, 256):
                t3 = time.perf_counter()
                dev_ids = m.generate_device(prompt, n_pred)
                dl.append(time.perf_counter() - t3)
            dev_s = min(dl[1], dl[3]) - min(dl[0], dl[2])
            m.set_timing(True)
            m.forward(prompt, n_past=0)
            attn_pf, _, _ = m.timing()
            m.set_timing(True)
            nxt = ids[0]
            for i in range(64):
                nxt, _ = m.forward([nxt], n_past=len(prompt) + i)
            attn_dec, _, _ = m.timing()
            m.set_timing(False)
            out[key] = {"prefill_ms": round((t1 - t0) * 1e3, 3),
                        "decode_tok_per_s": round(255 / (t2 - t1), 1),
                        "decode_ms_per_token": round((t2 - t1) * 1e3 / 255, 4),
                        "device_loop_decode_tok_per_s": round(255 / dev_s, 1),
                        "device_loop_ids_equal": dev_ids == ids,
                        "attn_us_per_token": round(attn_dec * 1e3 / 64, 2),
                        "prefill_attn_us": round(attn_pf * 1e3, 1),
                        "ids_equal_reference": ids == gold["ids"],
                        "ids_agree_steps": next((i for i, (a, b) in enumerate(zip(ids, gold["ids"]))
                                                 if a != b), len(ids))}
            free[key] = ids
        # the fused engine in lockstep with the reference-order one under
        # teacher forcing: where and by how much its argmax flips
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_FUSED)
        with Qwen2(path, n_ctx=2048, max_tokens=len(prompt)) as ref:
            ref.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
            recs = teacher_forced(m, ref, prompt, gold["ids"])
        summ = fork_summary(recs, free["fused"], gold["ids"])
        summ["reference_order_argmax_equal_reference"] = [r["ref_id"] for r in recs] == gold["ids"]
        summ["flips_are_near_ties"] = all(r["margin"] <= 2 * r["max_diff"] for r in recs
                                          if r["fused_id"] != r["ref_id"])
        out["fused"]["teacher_forced"] = {k: (round(v, 5) if isinstance(v, float) else v)
                                          for k, v in summ.items()}
    out["default_mode"] = "reference_order"  # the engine's default at n_ctx 2048: ids equal
    return out, path, d


def cpu_reference_engine(path, prompt_path, threads=16):
    """The reference CLI (oracle/_ref/mini_infer, built from the reference's own
    sources) with --bench on the host cores: prefill and decode tokens/s."""
    exe = os.path.join(ROOT, "oracle", "_ref", "mini_infer")
    if not os.path.exists(exe):
        return None
    import subprocess
    r = subprocess.run([exe, path, "--prompt-ids", prompt_path, "-c", "2048", "-n", "256", "-t",
                        str(threads), "--bench"], capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        return None
    kv = dict(t.split("=") for t in r.stdout.split())
    return {"prefill_tok_per_s": float(kv["prefill_tok_per_s"]),
            "decode_tok_per_s": float(kv["decode_tok_per_s"]), "threads": threads,
            "kind": "reference"}


def cpu_share():
    """Host cores this process may use: its affinity set, capped at
    OMP_NUM_THREADS and at 16 (one GPU's share of an 8-GPU MI355X host)."""
    try:
        allowed = len(os.sched_getaffinity(0))
    except OSError:
        allowed = os.cpu_count() or 1
    return max(1, min(allowed, int(os.environ.get("OMP_NUM_THREADS", "16") or 16), 16))


def cpu_info():
    """The host CPU: model string (with the family / model / stepping numbers,
    which name the part where a virtualised host shortens the string),
    logical CPUs (nproc), physical cores."""
    model, cores = "unknown", set()
    ids = {}
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model == "unknown":
                model = v
            elif k in ("vendor_id", "cpu family", "model", "stepping") and k not in ids:
                ids[k] = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
            elif not k and phys is not None and core is not None:
                cores.add((phys, core))
                phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    if ids:
        model += " (%s)" % ", ".join("%s %s" % (k, ids[k]) for k in ("vendor_id", "cpu family", "model", "stepping")
                                     if k in ids)
    return dict(cpu=model, nproc=os.cpu_count() or 1, physical_cores=len(cores) or None)


def cpu_baseline(n_layers_sample=24, n_kv=4096, target_s=12.0):
    """The reference three-node CPU path (attn_qk -> softmax -> attn_kqv as
    graph nodes on its own thread pool) on the host cores, on a bounded sample
    of the decode workload: 24 layers' decode attention at n_kv = 4096. Thread
    counts 1, 2, 4, ... up to the job's CPU share are swept as the reference's
    scripts/bench_threads.py sweeps them (1 warmup, median of 5); the best is
    then timed over about `target_s` seconds of CPU work (median pass), and
    prefill-1024 a few times."""
    import numpy as np
    from oracle import cpu_attention
    impl = cpu_attention.reference() or cpu_attention.oracle()
    share = cpu_share()
    rng = np.random.default_rng(7)
    qs = [rng.standard_normal((1, 14, 64), dtype=np.float32) for _ in range(n_layers_sample)]
    ks = [rng.standard_normal((n_kv, 2, 64), dtype=np.float32) for _ in range(n_layers_sample)]
    vs = [rng.standard_normal((n_kv, 2, 64), dtype=np.float32) for _ in range(n_layers_sample)]
    nbytes = decode_bytes(n_layers_sample, n_kv, 14, 2, 64, 4)
    counts = sorted({min(1 << i, share) for i in range(6)} | {share})
    sweep = {}
    for t in counts:
        ts, _ = impl.time_attention(qs, ks, vs, n_kv - 1, 0.125, t, warmup=1, reps=5)
        sweep[t] = nbytes / ts / 1e9
    threads = max(sweep, key=sweep.get)
    t0, _ = impl.time_attention(qs, ks, vs, n_kv - 1, 0.125, threads, warmup=1, reps=3)
    reps = int(min(5000, max(7, target_s / max(t0, 1e-6))))
    t, _ = impl.time_attention(qs, ks, vs, n_kv - 1, 0.125, threads, warmup=0, reps=reps)
    # prefill-1024 on the CPU (the reference computes every key, masked or
    # not; the FLOP count below is still the causal one)
    q = rng.standard_normal((1024, 14, 64), dtype=np.float32)
    k = rng.standard_normal((1024, 2, 64), dtype=np.float32)
    v = rng.standard_normal((1024, 2, 64), dtype=np.float32)
    tp, _ = impl.time_attention([q], [k], [v], 0, 0.125, threads, warmup=1, reps=5)
    info = cpu_info()
    return dict(value=nbytes / t / 1e9, unit="GB/s", cores=threads, kind=impl.kind,
                sample=f"24 layers x decode n_kv=4096 (14 Q / 2 KV heads, head_dim 64, F32), "
                       f"median of {reps} passes ({reps * t:.1f} s) at the best thread count; "
                       f"attn_qk -> softmax -> attn_kqv, barrier per node, static (head,row) split",
                us_per_layer=t * 1e6 / n_layers_sample,
                prefill1024_s=tp, prefill1024_tflops=causal_flops(1024, 14, 64) / tp / 1e12,
                threads_sweep_gbps={str(k): round(v, 3) for k, v in sweep.items()},
                best_threads=threads, cpu_share=share, **info)


def measured_mfma():
    """Matrix-core use of the prefill kernel from the committed rocprofv3
    counter summary (profiles/prefill_mfma.txt): float products at n=1024
    and 4096, split bf16 pairs at n=1024."""
    p = os.path.join(ROOT, "profiles", "prefill_mfma.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        m = json.load(f)
    keep = ("kernel_us", "mfma_insts", "issued_flops", "issued_tflops", "issued_peak_tflops", "issued_frac_of_peak",
            "mfma_busy_frac", "causal_frac_of_issued_peak")
    return {"source": "profiles/prefill_mfma.txt (SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_VALU_MFMA_MOPS_F32/_BF16, "
                      "kernel trace)",
            **{k: {f: v[f] for f in keep if f in v} for k, v in m.items()}}


def measured_traffic(name="decode_traffic.json"):
    """HBM bytes per launch from a committed rocprofv3 PMC summary."""
    p = os.path.join(ROOT, "profiles", name)
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build runs "
              "every kernel on a single MI355X and has no multi-GPU path.", file=sys.stderr)
        sys.exit(2)
    import torch
    import mi_hip_attn as mh
    lib = mh.lib()
    lib.init(0)
    if args.nondeterministic:
        lib.check(lib.mi_hip_set_deterministic(0))
    torch.cuda.set_device(0)
    stream = torch.cuda.current_stream().cuda_stream
    only = set(filter(None, args.only.split(",")))
    want = lambda k: not only or k in only

    res = {}
    if want("decode"):
        res["decode"] = bench_decode(torch, mh, lib, stream, args.steps, args.warmup)
        # the other kernels on the same workload (the default for an F32 cache
        # is the vector-unit kernel with its LDS ring)
        for key, mode in (("decode_matrix", mh.MI_HIP_DECODE_MATRIX), ("decode_stream", mh.MI_HIP_DECODE_STREAM)):
            lib.check(lib.mi_hip_set_decode_mode(mode))
            res[key] = bench_decode(torch, mh, lib, stream, args.steps, args.warmup)
        lib.check(lib.mi_hip_set_decode_mode(mh.MI_HIP_DECODE_AUTO))
        print(f"# decode 24x4096: vector units (default) {res['decode']['kernel_ms'] * 1e3:.2f} us, streaming "
              f"kernel {res['decode_stream']['kernel_ms'] * 1e3:.2f} us, matrix cores "
              f"{res['decode_matrix']['kernel_ms'] * 1e3:.2f} us", file=sys.stderr, flush=True)
        res["read_floor"] = bench_read_floor(torch, lib, stream, args.steps, args.warmup,
                                             24 * 2 * 4096 * 2 * 64 * 4)
        print(f"# read floor of the step's 100.7 MB: {res['read_floor']['us']:.2f} us "
              f"({res['read_floor']['gbps']:.1f} GB/s)", file=sys.stderr, flush=True)
    if want("streams"):
        res["streams"] = bench_decode_streams(torch, mh, lib, args.steps, args.warmup)
        print(f"# decode 24x4096 over 2 streams: {res['streams']['gbps']:.1f} GB/s "
              f"({res['streams']['us_per_launch']:.2f} us per launch)", file=sys.stderr, flush=True)
        print(f"# decode 24x4096: {res['decode']['gbps']:.1f} GB/s per step, kernel "
              f"{res['decode']['kernel_gbps']:.1f} GB/s", file=sys.stderr, flush=True)
    if want("sweep"):
        res["sweep"] = {}
        for n_kv in (128, 1024, 4096, 16384, 32768):
            st = max(20, min(args.steps, 8_000_000 // (n_kv * 24)))
            res["sweep"][n_kv] = (res["decode"] if n_kv == 4096 and "decode" in res else
                                  bench_decode(torch, mh, lib, stream, st, max(2, st // 10), n_kv=n_kv))
            print(f"# decode 24x{n_kv}: {res['sweep'][n_kv]['kernel_gbps']:.1f} GB/s, "
                  f"{res['sweep'][n_kv]['kernel_ms'] * 1e3:.2f} us", file=sys.stderr, flush=True)
        res["config1"] = bench_decode(torch, mh, lib, stream, args.steps, args.warmup, n_layers=1,
                                      n_kv=512)
        print(f"# decode 1 layer x 512: {res['config1']['kernel_ms'] * 1e3:.2f} us", file=sys.stderr,
              flush=True)
    if want("prefill"):
        res["prefill1024"] = bench_prefill(torch, mh, lib, stream, args.steps, args.warmup, 1024)
        res["prefill4096"] = bench_prefill(torch, mh, lib, stream, max(10, args.steps // 10),
                                           max(2, args.warmup // 10), 4096)
        # the split-bf16 form beside the default float products
        lib.check(lib.mi_hip_set_prefill_mode(mh.MI_HIP_PREFILL_SPLIT_BF16))
        res["prefill1024_split"] = bench_prefill(torch, mh, lib, stream, args.steps, args.warmup, 1024)
        lib.check(lib.mi_hip_set_prefill_mode(mh.MI_HIP_PREFILL_AUTO))
        # an F16 cache at the same shape (the default form for it: f16
        # products, exact in the cache operand)
        res["prefill1024_f16"] = bench_prefill(torch, mh, lib, stream, args.steps, args.warmup, 1024, f16=True)
        print(f"# prefill 1024: {res['prefill1024']['tflops']:.2f} TF/s, 4096: "
              f"{res['prefill4096']['tflops']:.2f} TF/s; F16 cache 1024: "
              f"{res['prefill1024_f16']['tflops']:.2f} TF/s", file=sys.stderr, flush=True)
    if want("d7b"):
        res["decode7b"] = bench_decode(torch, mh, lib, stream, args.steps, args.warmup,
                                       n_layers=1, n_kv=8192, h=28, hkv=4, d=128, f16=True)
        print(f"# decode 7B F16 8192: {res['decode7b']['kernel_gbps']:.1f} GB/s", file=sys.stderr,
              flush=True)
    if want("perlayer"):
        res["per_layer"] = bench_decode_per_layer(torch, mh, lib, stream, args.steps, args.warmup)
        print(f"# per-layer launches: {res['per_layer']['us_per_layer']:.2f} us/layer",
              file=sys.stderr, flush=True)

    if want("q8"):
        res["q8"] = bench_q8_matvec(torch, mh, lib, stream, args.steps, args.warmup)
        print(f"# q8_0 matvec 151936x896: {res['q8']['gbps']:.1f} GB/s "
              f"({res['q8']['kernel_ms'] * 1e3:.2f} us)", file=sys.stderr, flush=True)

    if want("e2e"):
        res["e2e"], e2e_model, e2e_dir = bench_e2e(mh)
        r, f = res["e2e"]["reference_order"], res["e2e"]["fused"]
        print(f"# e2e 0.5B Q8_0 (default reference-order attention): decode {r['decode_tok_per_s']} tok/s "
              f"(device loop {r['device_loop_decode_tok_per_s']}), ids equal: {r['ids_equal_reference']}, "
              f"attention {r['attn_us_per_token']} us/token; fused: {f['decode_tok_per_s']} tok/s, "
              f"attention {f['attn_us_per_token']} us/token", file=sys.stderr, flush=True)
        if not args.no_cpu:
            import qwen2_gguf as gg
            ids_path = os.path.join(e2e_dir, "ids.txt")
            with open(ids_path, "w") as fh:
                fh.write(" ".join(map(str, gg.prompt_ids(E2E_SEED, 128, gg.QWEN2_05B["n_vocab"]))))
            res["e2e"]["cpu_reference_engine"] = cpu_reference_engine(e2e_model, ids_path)
        import shutil
        shutil.rmtree(e2e_dir, ignore_errors=True)

    if want("memread"):
        res["memread"] = bench_memread(torch, lib, stream, 20, 3)
        res["memread"].update(device_info())
        print(f"# read ceiling 1 GiB: {res['memread']['gbps']:.1f} GB/s "
              f"(by workgroup count: {res['memread']['gbps_by_workgroups']}); rocminfo: "
              f"{res['memread']['cus']} CUs, {res['memread']['max_clock_mhz']} MHz", file=sys.stderr,
              flush=True)

    if "copy" in only:
        res["copy"] = bench_copy(torch, max(5, args.steps // 10), 2)
        print(f"# copy 256 MiB: {res['copy']['gbps']:.1f} GB/s (read + write)", file=sys.stderr,
              flush=True)

    cpu = None
    if not args.no_cpu:
        t0 = time.time()
        cpu = cpu_baseline()
        print(f"# cpu baseline {cpu['value']:.2f} GB/s ({time.time() - t0:.1f}s)", file=sys.stderr,
              flush=True)

    d = res.get("decode")
    out = {
        "metric": METRIC,
        "value": round(d["gbps"], 2) if d else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 6) if d else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) Q/K/V generated on the device",
        "config": {
            "workload": "decode attention: 24 independent layer caches x n_kv=4096, 1 query "
                        "token, 14 Q / 2 KV heads (GQA 7), head_dim 64, F32 K/V, one batched "
                        "launch per step, cache sets rotated beyond the 256 MB MALL",
            "spinup_s": SPINUP_S,
            "n_layers": 24, "n_kv": 4096, "n_head": 14, "n_head_kv": 2, "head_dim": 64,
            "cache_sets": d["sets"] if d else None,
        },
    }
    if d:
        out["roofline"] = {
            "bound": "hbm", "achieved": round(d["kernel_gbps"], 2), "peak": HBM_PEAK_GBPS,
            "unit": "GB/s", "frac": round(d["kernel_gbps"] / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(),
            "bytes_per_launch": d["bytes"], "kernel_us": round(d["kernel_ms"] * 1e3, 3),
        }
        if "decode_matrix" in res:
            dm, dr = res["decode_matrix"], res["decode_stream"]
            out["roofline"]["kernel"] = ("decode_kernel, vector units (float products, no MFMA; "
                                         "MI_HIP_DECODE_VALU, the default for an F32 cache)")
            out["decode_matrix_24x4096"] = {
                "what": "the same step on the matrix-core form (split-bf16 products, MI_HIP_DECODE_MATRIX)",
                "us": round(dm["kernel_ms"] * 1e3, 3), "gbps": round(dm["kernel_gbps"], 1),
                "frac": round(dm["kernel_gbps"] / HBM_PEAK_GBPS, 4)}
            out["decode_stream_24x4096"] = {
                "what": "the same step on the streaming vector-unit kernel (MI_HIP_DECODE_STREAM: K/V straight "
                        "into registers, last-arriver merge)",
                "us": round(dr["kernel_ms"] * 1e3, 3), "gbps": round(dr["kernel_gbps"], 1),
                "frac": round(dr["kernel_gbps"] / HBM_PEAK_GBPS, 4)}
        if "read_floor" in res:
            rf = res["read_floor"]
            out["roofline"]["read_floor"] = {
                "what": "mi_hip_memread (nontemporal 16-byte loads, as the decode kernel's) over exactly the "
                        "step's 100,663,296 cache bytes, 7 buffers rotated, back to back; fastest workgroup count",
                "us": round(rf["us"], 3), "gbps": round(rf["gbps"], 1),
                "frac_of_peak": round(rf["gbps"] / HBM_PEAK_GBPS, 4), "workgroups": rf["workgroups"],
                "us_by_workgroups": rf["us_by_workgroups"],
                "decode_over_floor_us": round(d["kernel_ms"] * 1e3 - rf["us"], 3)}
        if "memread" in res:
            m = res["memread"]
            out["roofline"]["measured_read_ceiling"] = {
                "gbps": round(m["gbps"], 1), "frac_of_peak": round(m["gbps"] / HBM_PEAK_GBPS, 4),
                "achieved_frac_of_ceiling": round(d["kernel_gbps"] / m["gbps"], 4),
                "workload": f"mi_hip_memread: load-and-accumulate pass over 1 GiB, {m['n_sums']} "
                            "workgroups of 512 (the fastest of 1024-16384)",
                "cus": m["cus"], "max_clock_mhz": m["max_clock_mhz"]}
    if cpu:
        out["cpu_baseline"] = {k: (round(v, 4) if isinstance(v, float) else v)
                               for k, v in cpu.items()}
    if "q8" in res:
        q8 = res["q8"]
        out["q8_0_matvec"] = {
            "metric": "MUL_MAT Q8_0 weights x 1 token GB/s (Qwen2.5-0.5B output projection, "
                      "151936 x 896)",
            "gbps": round(q8["gbps"], 2), "us": round(q8["kernel_ms"] * 1e3, 2),
            "roofline": {"bound": "hbm", "achieved": round(q8["gbps"], 2), "peak": HBM_PEAK_GBPS,
                         "unit": "GB/s", "frac": round(q8["gbps"] / HBM_PEAK_GBPS, 4),
                         "traffic": measured_traffic("q8_0_matvec_traffic.json"),
                         "bytes_per_launch": q8["bytes"]},
        }
    if "prefill1024" in res:
        p1, p4 = res["prefill1024"], res["prefill4096"]
        mm = measured_mfma()
        # FLOPs the launch issues on the matrix cores (the causal count plus the
        # diagonal tiles' masked halves), from the instruction counters; the
        # same in every launch of this shape
        issued = (mm or {}).get("f32_1024", {}).get("issued_flops")
        out["prefill"] = {
            "metric": "prefill-1024 causal attn TFLOP/s (14 Q / 2 KV heads, head_dim 64, F32)",
            "products": "f32 (v_mfma_f32_32x32x2f32, the issued type)",
            "tflops_1024": round(p1["tflops"], 2), "us_1024": round(p1["kernel_ms"] * 1e3, 2),
            "tflops_4096": round(p4["tflops"], 2), "us_4096": round(p4["kernel_ms"] * 1e3, 2),
            "roofline": {"bound": "mfma", "achieved": round(p1["tflops"], 2),
                         "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(p1["tflops"] / FP32_MFMA_PEAK_TFLOPS, 4),
                         "flops_per_launch": p1["flops"],
                         "issued_flops_per_launch": issued,
                         "issued_tflops": round(issued / p1["kernel_ms"] / 1e9, 2) if issued else None,
                         "issued_frac": (round(issued / p1["kernel_ms"] / 1e9 / FP32_MFMA_PEAK_TFLOPS, 4)
                                         if issued else None),
                         "mfma_counters": mm},
        }
        if "prefill1024_split" in res:
            ps = res["prefill1024_split"]
            # three bf16 products per float product: the issued bf16 FLOPs (from
            # the instruction counters) are ~3.09x the causal count, with the
            # diagonal tiles' masked halves
            iss = (mm or {}).get("split_1024", {}).get("issued_flops") or 3 * ps["flops"]
            out["prefill"]["split_bf16_1024"] = {
                "tflops_causal": round(ps["tflops"], 2), "us": round(ps["kernel_ms"] * 1e3, 2),
                "issued_flops_per_launch": iss,
                "issued_tflops_bf16": round(iss / ps["kernel_ms"] / 1e9, 2),
                "frac_of_bf16_peak": round(iss / ps["kernel_ms"] / 1e9 / BF16_MFMA_PEAK_TFLOPS, 4)}
        if "prefill1024_f16" in res:
            pf = res["prefill1024_f16"]
            # two f16 products per product step (Q and P as f16 pairs) over the
            # same tiles as the float form: twice its issued FLOPs (the
            # instruction counters give the same)
            iss = ((mm or {}).get("f16_cache_1024", {}).get("issued_flops")
                   or (2 * issued if issued else 2 * 1.03 * pf["flops"]))
            out["prefill"]["f16_cache_1024"] = {
                "products": "f16 (v_mfma_f32_32x32x16_f16; the cache operand exact, Q and P as f16 pairs)",
                "tflops_causal": round(pf["tflops"], 2), "us": round(pf["kernel_ms"] * 1e3, 2),
                "issued_flops_per_launch": iss,
                "issued_tflops_f16": round(iss / pf["kernel_ms"] / 1e9, 2),
                "frac_of_f16_peak": round(iss / pf["kernel_ms"] / 1e9 / BF16_MFMA_PEAK_TFLOPS, 4)}
    if "sweep" in res:
        out["decode_sweep"] = {
            "workload": "24 independent layer caches, 1 query token, 14 Q / 2 KV heads, head_dim 64, "
                        "F32 K/V, one batched launch per step, cache sets rotated beyond the MALL",
            "by_n_kv": {str(n): {"us": round(r["kernel_ms"] * 1e3, 3), "us_per_layer":
                                 round(r["kernel_ms"] * 1e3 / 24, 3), "gbps": round(r["kernel_gbps"], 1),
                                 "frac": round(r["kernel_gbps"] / HBM_PEAK_GBPS, 4),
                                 "bytes": r["bytes"], "cache_sets": r["sets"]}
                        for n, r in res["sweep"].items()}}
        c1 = res["config1"]
        out["decode_config1"] = {
            "workload": "one layer, n_kv 512, 14 Q / 2 KV heads, head_dim 64, F32 K/V (the reference's "
                        "CPU-runnable case)",
            "us_per_layer": round(c1["kernel_ms"] * 1e3, 3), "gbps": round(c1["kernel_gbps"], 1),
            "frac": round(c1["kernel_gbps"] / HBM_PEAK_GBPS, 4), "bytes": c1["bytes"]}
    if "decode7b" in res:
        r = res["decode7b"]
        out["decode_7b_f16"] = {"n_kv": 8192, "gbps": round(r["kernel_gbps"], 1),
                                "us": round(r["kernel_ms"] * 1e3, 2),
                                "frac": round(r["kernel_gbps"] / HBM_PEAK_GBPS, 4)}
    if "per_layer" in res:
        out["decode_per_layer_launch"] = {k: round(v, 3) for k, v in res["per_layer"].items()}
    if "streams" in res:
        sr = res["streams"]
        out["decode_two_streams"] = {
            "what": "the same 24 x 4096 launches alternating over two streams (independent batches, one "
                    "workspace per stream): launches overlap, so one's start hides another's tail",
            "us_per_launch": round(sr["us_per_launch"], 3), "gbps": round(sr["gbps"], 1),
            "frac_of_8tbs": round(sr["gbps"] / 8000.0, 4), "early_fallbacks": sr["early_fallbacks"],
            "lost_groups": sr["lost_groups"]}
    if "e2e" in res:
        out["e2e_qwen05_q8_0"] = res["e2e"]
    print(json.dumps(out))


if __name__ == "__main__":
    main()
