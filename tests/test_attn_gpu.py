"""GPU parity of the fused decode and prefill kernels against the oracle.

Bar (written here, from the task's stated tolerance): |gpu - ref| <=
1e-4 + 1e-4*|ref| for F32 K/V; 1e-2 for F16 K/V against unrounded inputs.
With an F16 cache the oracle runs the engine's F32 ops on the exactly widened
cache, and then the F32 bar applies too.
"""
import ctypes

import numpy as np
import pytest

from conftest import TOL_F16, TOL_F32, case_inputs, load_golden
from oracle import cpu_attention
import mi_hip_attn as mh

pytestmark = pytest.mark.gpu


def assert_close(got, want, tol, what=""):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = tol["atol"] + tol["rtol"] * np.abs(want.astype(np.float64))
    worst = float((err / bound).max()) if err.size else 0.0
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert worst <= 1.0, f"{what}: max abs err {err.max():.3e}, worst err/bound {worst:.3f}"


def dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def fused(hip, stream, q, k, v, n_past, scale, f16=False, ws=None):
    """Runs mi_hip_attn_fwd on explicit device tensors (with the decode
    workspace `ws`, else the library's); returns host output."""
    import torch
    assert k.shape == v.shape and k.shape[2] == q.shape[2] and q.shape[1] % k.shape[1] == 0
    assert n_past + q.shape[0] <= k.shape[0]
    dq = dev(q)
    dk = dev(k.astype(np.float16)) if f16 else dev(k)
    dv = dev(v.astype(np.float16)) if f16 else dev(v)
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
    a = mh.attn_args(dq, out, q.shape[1] // k.shape[1], n_past, scale, stream, k=dk, v=dv, ws=ws)
    hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def ref_out(oracle, q, k, v, n_past, scale, f16=False, threads=16):
    if f16:
        k = cpu_attention.fp16_widen(k.astype(np.float16))
        v = cpu_attention.fp16_widen(v.astype(np.float16))
    return oracle.attention(q, k, v, n_past, scale, threads)[2]


def test_golden_cases(hip, stream, golden_manifest, decode_mode):
    for name, c in golden_manifest["cases"].items():
        if c["head_dim"] not in (64, 128):
            continue  # head_dim 4 (tiny model) runs through the node operators
        print("case", name, flush=True)
        q, k, v = case_inputs(c)
        f16 = c["kv_type"] == "f16"
        got = fused(hip, stream, q, k, v, c["n_past"], c["scale"], f16)
        assert_close(got, load_golden(name)["out"], TOL_F32, name)
        if f16:
            unrounded = cpu_attention.oracle().attention(q, k, v, c["n_past"], c["scale"], 4)[2]
            assert_close(got, unrounded, TOL_F16, name + " vs F32 inputs")


@pytest.mark.parametrize("n_kv", [1, 63, 64, 65, 128, 1000, 1024, 4096, 16384, 32768])
def test_decode_sweep_qwen05_shape(hip, stream, oracle, n_kv, decode_mode):
    print("decode n_kv", n_kv, flush=True)
    q, k, v = cpu_attention.make_inputs(1236 + n_kv, 64, 14, 2, n_kv, 1)
    got = fused(hip, stream, q, k, v, n_kv - 1, 0.125)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, 0.125), TOL_F32, f"n_kv={n_kv}")


# More than 8 Q heads per KV head go in ceil(n_rep / 8) chunks cut as evenly
# as they can be, whatever n_rep's divisors (9 -> 4 + 5, 11 -> 5 + 6,
# 13 -> 6 + 7, 15 -> 7 + 8, 17 -> 5 + 6 + 6), at short and long contexts.
@pytest.mark.parametrize("n_rep,hkv,d", [(1, 4, 64), (2, 2, 64), (4, 2, 128), (8, 2, 64),
                                         (3, 2, 64), (6, 1, 128), (14, 1, 64), (9, 2, 64),
                                         (11, 2, 64), (13, 1, 128), (15, 2, 64), (16, 2, 128),
                                         (17, 1, 64), (24, 1, 64)])
@pytest.mark.parametrize("n_kv", [777, 5000])
def test_decode_group_shapes(hip, stream, oracle, n_rep, hkv, d, n_kv, decode_mode):
    q, k, v = cpu_attention.make_inputs(31 + n_rep, d, n_rep * hkv, hkv, n_kv, 1)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_kv - 1, scale)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale), TOL_F32)


# Short contexts, where every group gets one workgroup: the vector kernel then
# cuts groups of more than 4 heads into two chunks (7 -> 3 + 4, 5 -> 2 + 3,
# 14 -> four chunks of 3 or 4), as it does for launches whose groups merge
# parts when the split keeps their part counts (n_kv 383..4096 here, early and
# flat merges: each chunk's parts merge among themselves); with kpg forced to 1
# the groups stay whole.
@pytest.mark.parametrize("n_rep,hkv,d,n_kv", [(5, 2, 64, 200), (6, 2, 128, 100), (7, 2, 64, 130),
                                              (7, 2, 64, 383), (8, 1, 64, 17), (14, 2, 64, 256),
                                              (16, 1, 128, 64), (7, 2, 64, 512), (7, 2, 64, 1000),
                                              (5, 2, 64, 777), (14, 2, 64, 700), (7, 2, 64, 2048),
                                              (7, 2, 64, 4096), (7, 1, 64, 3000)])
@pytest.mark.parametrize("kpg", [0, 1])
def test_decode_short_context_head_chunks(hip, stream, oracle, tuning, n_rep, hkv, d, n_kv, kpg,
                                          decode_mode):
    print("short decode", n_rep, hkv, d, n_kv, kpg, flush=True)
    tuning(kpg=kpg)
    q, k, v = cpu_attention.make_inputs(5150 + 3 * n_rep + d + n_kv, d, n_rep * hkv, hkv, n_kv, 1)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_kv - 1, scale)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale), TOL_F32)


# Every F16-cache kernel variant: head_dim 64 (8 waves, 4-slot ring) with
# groups over and under 4 heads, head_dim 128 with groups of at most 4 (one
# head slot per row, 64 KB ring) and over 4; the Qwen2.5-0.5B shape at short,
# odd and long contexts.
@pytest.mark.parametrize("n_rep,hkv,d,n_kv", [(1, 4, 64, 777), (2, 2, 128, 777), (4, 2, 128, 777),
                                              (7, 2, 64, 1), (7, 2, 64, 17), (7, 2, 64, 777),
                                              (7, 2, 64, 4096), (8, 1, 128, 2000)])
def test_decode_f16_cache_shapes(hip, stream, oracle, n_rep, hkv, d, n_kv, decode_mode):
    print("f16 decode", n_rep, hkv, d, n_kv, flush=True)
    q, k, v = cpu_attention.make_inputs(900 + 7 * n_rep + d + n_kv, d, n_rep * hkv, hkv, n_kv, 1)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_kv - 1, scale, f16=True)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale, f16=True), TOL_F32, "widened")
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale), TOL_F16, "unrounded")


# The library's own choice for an F16 cache (MI_HIP_DECODE_AUTO, no fixture):
# heads split on the vector units where the split launch's waves stream fewer
# than 4 sub-tiles (one layer of the 0.5B shape at n_kv 512-8192, the 7B shape
# at 512), whole on the matrix cores otherwise (32768; the 7B shape at 4096
# and 8192).
@pytest.mark.parametrize("n_rep,hkv,d,n_kv", [(7, 2, 64, 512), (7, 2, 64, 1024), (7, 2, 64, 4096),
                                              (7, 2, 64, 8192), (7, 2, 64, 32768), (7, 4, 128, 512),
                                              (7, 4, 128, 4096), (7, 4, 128, 8192)])
def test_decode_f16_cache_default_choice(hip, stream, oracle, n_rep, hkv, d, n_kv):
    print("f16 decode, default kernel choice", n_rep, hkv, d, n_kv, flush=True)
    q, k, v = cpu_attention.make_inputs(1900 + n_kv + d, d, n_rep * hkv, hkv, n_kv, 1)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_kv - 1, scale, f16=True)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale, f16=True), TOL_F32, "widened")
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale), TOL_F16, "unrounded")


@pytest.fixture(params=[mh.MI_HIP_DECODE_MATRIX, mh.MI_HIP_DECODE_VALU, mh.MI_HIP_DECODE_STREAM],
                ids=["matrix", "valu", "stream"])
def decode_mode(request, hip):
    """Runs a decode test on each decode kernel (matrix cores, vector units);
    the library default picks one of them per launch."""
    hip.check(hip.mi_hip_set_decode_mode(request.param))
    yield request.param
    hip.check(hip.mi_hip_set_decode_mode(mh.MI_HIP_DECODE_AUTO))


def test_decode_f16_cache_large_queries(hip, stream, oracle, decode_mode):
    # Queries far outside the f16 range (|q| up to ~4e5 on some heads, others
    # unscaled): the matrix kernel scales such a head's f16 operand by a power
    # of two and undoes it on the scores; the result must not change.
    n_kv, d = 1500, 128
    q, k, v = cpu_attention.make_inputs(4242, d, 8, 2, n_kv, 1)
    q = q.copy()
    q[0, 1] *= 1e5
    q[0, 6] *= 3e4
    q[0, 7] *= 50.0
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_kv - 1, scale, f16=True)
    assert np.isfinite(got).all()
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale, f16=True), TOL_F32, "widened")


@pytest.fixture()
def tuning(hip):
    """Sets decode planner knobs for one test and restores the defaults."""
    def set_(kpg=-1, early=-1, solo=-1, claim=-1, det=None):
        hip.check(hip.mi_hip_decode_tuning(kpg, early, solo, claim))
        if det is not None:
            hip.check(hip.mi_hip_set_deterministic(det))
    yield set_
    hip.check(hip.mi_hip_decode_tuning(0, 1, 1, 0))
    hip.check(hip.mi_hip_set_deterministic(1))


# Forced workgroups per group: the early protocol (2..8 parts, with and without
# a part that gets no sub-tile), one team (9..32 parts) and several teams
# (more than 32 parts at head_dim 64, more than 8 at head_dim 128).
@pytest.mark.parametrize("kpg,early", [(2, 1), (5, 1), (8, 1), (8, 0), (9, 1), (24, 0), (40, 1), (100, 0)])
@pytest.mark.parametrize("d,f16", [(64, False), (128, True)])
@pytest.mark.parametrize("claim", [1, 0])
def test_decode_forced_split(hip, stream, oracle, tuning, kpg, early, d, f16, claim, decode_mode):
    # claim 1: sub-tiles claimed from the group counter (dynamic takes, which
    # the deterministic mode turns off); 0: every kpg-th sub-tile per part,
    # in fixed (deterministic) order
    print("forced split", kpg, early, d, f16, claim, flush=True)
    tuning(kpg=kpg, early=early, claim=claim, det=0 if claim else 1)
    n_kv = 3000 + 20 * kpg  # long enough that the forced split is not capped below 33 parts
    hkv = 2 if d == 64 else 4
    q, k, v = cpu_attention.make_inputs(4100 + kpg + d, d, 7 * hkv, hkv, n_kv, 1)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_kv - 1, scale, f16=f16)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale, f16=f16), TOL_F32)


# The flat merge (more than 8 parts, launch resident at once): every part
# merges its slice of the output over all parts' records. One KV head group, so
# that up to 256 parts fit the device: 2..64 lanes per pair (one wave) and
# 128/256 (waves meeting in LDS).
@pytest.mark.parametrize("d,f16,kpg", [(64, False, 9), (64, False, 33), (64, False, 100), (64, False, 256),
                                       (128, True, 64), (128, True, 129), (128, True, 256)])
def test_decode_flat_merge(hip, stream, oracle, tuning, d, f16, kpg, decode_mode):
    print("flat merge", d, f16, kpg, flush=True)
    tuning(kpg=kpg, early=1)
    waves = 8 if d == 64 else 4
    n_kv = 16 * waves * kpg + 37  # every wave of every part has a sub-tile, the last one partial
    q, k, v = cpu_attention.make_inputs(8800 + kpg + d, d, 7, 1, n_kv, 1)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    ws = hip.workspace_create(1, 7, d)
    try:
        got = fused(hip, stream, q, k, v, n_kv - 1, scale, f16=f16, ws=ws)
        rc, fallbacks, lost = hip.workspace_check(ws, stream)
        assert rc == 0 and lost == 0 and fallbacks == 0
    finally:
        hip.check(hip.mi_hip_workspace_destroy(ws))
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale, f16=f16), TOL_F32)


def test_flat_merge_fallback_is_exact(hip, stream, oracle, tuning):
    # 24 items x 2 groups x 24 parts = 1152 workgroups (one per CU at a time)
    # with the flat merge forced: a group that straddles the resident set (48
    # workgroups per item do not divide the CU count) has parts that run out
    # of polls (limit 0) while others have not started; they mark the start
    # counter and leave their slices to the last part to start, which merges
    # every slice. Groups resident as a whole keep waiting. Exact either way.
    import torch
    tuning(kpg=24, early=2)
    ws = hip.workspace_create(2, 14, 64)
    try:
        hip.check(hip.mi_hip_workspace_set_poll_limit(ws, 0))
        total = 0
        for rep in range(3):
            ins, outs, _ = batch_24(hip, stream, 4096, 9100 + 100 * rep, ws=ws)
            torch.cuda.synchronize()
            check_batch_24(oracle, ins, outs, 4096, f"rep {rep}")
            rc, fallbacks, lost = hip.workspace_check(ws, stream)
            print("1152 workgroups: fallbacks", fallbacks, "lost", lost, flush=True)
            assert rc == 0 and lost == 0
            total += fallbacks
        assert total > 0
    finally:
        hip.check(hip.mi_hip_workspace_destroy(ws))


@pytest.fixture()
def deterministic(hip):
    """Deterministic fused kernels (the library default) for one test."""
    hip.check(hip.mi_hip_set_deterministic(1))
    yield
    hip.check(hip.mi_hip_set_deterministic(1))


@pytest.fixture()
def dynamic_takes(hip):
    """The non-deterministic (counter-taking) fused kernels for one test."""
    hip.check(hip.mi_hip_set_deterministic(0))
    yield
    hip.check(hip.mi_hip_set_deterministic(1))


@pytest.mark.parametrize("kpg", [0, 3, 8, 24])
def test_deterministic_decode_repeats_bit_for_bit(hip, stream, oracle, tuning, deterministic, kpg, decode_mode):
    # With fixed per-wave takes every merge runs in a fixed order, so five
    # launches of one problem give the same bits (planned split and forced
    # splits over both merge protocols), and they meet the oracle's bar.
    tuning(kpg=kpg)
    n_kv = 4096 + 77
    q, k, v = cpu_attention.make_inputs(6060 + kpg, 64, 14, 2, n_kv, 1)
    runs = [fused(hip, stream, q, k, v, n_kv - 1, 0.125) for _ in range(5)]
    for i, r in enumerate(runs[1:]):
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32)), f"run {i + 1}"
    assert_close(runs[0], ref_out(oracle, q, k, v, n_kv - 1, 0.125), TOL_F32)


def test_prefill_dynamic_takes(hip, stream, oracle, dynamic_takes):
    # the counter-taking prefill (deterministic mode off) against the oracle
    n = 1024
    q, k, v = cpu_attention.make_inputs(6262, 64, 14, 2, n, n)
    got = fused(hip, stream, q, k, v, 0, 0.125)
    for j in (0, 33, 640, 1023):
        want = oracle.attention(q[j:j + 1], k, v, j, 0.125, 8)[2]
        assert_close(got[j:j + 1], want, TOL_F32, f"row {j}")


def test_deterministic_prefill_repeats_bit_for_bit(hip, stream, oracle, deterministic):
    n = 1024
    q, k, v = cpu_attention.make_inputs(6161, 64, 14, 2, n, n)
    runs = [fused(hip, stream, q, k, v, 0, 0.125) for _ in range(3)]
    for i, r in enumerate(runs[1:]):
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32)), f"run {i + 1}"
    for j in (0, 31, 500, 1023):
        want = oracle.attention(q[j:j + 1], k, v, j, 0.125, 8)[2]
        assert_close(runs[0][j:j + 1], want, TOL_F32, f"row {j}")


def test_decode_back_to_back_launches_share_no_records(hip, stream, oracle):
    # Two launches of one shape on one stream, no synchronisation between them:
    # they use the same cross-workgroup record slots, and the second must merge
    # only its own records (a record of the first launch carries an older stamp).
    import torch
    n_kv = 4096
    runs = []
    for seed in (71, 72):
        q, k, v = cpu_attention.make_inputs(seed, 64, 14, 2, n_kv, 1)
        out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
        dq, dk, dv = dev(q), dev(k), dev(v)
        runs.append((q, k, v, out, dq, dk, dv))
    for q, k, v, out, dq, dk, dv in runs:
        a = mh.attn_args(dq, out, 7, n_kv - 1, 0.125, stream, k=dk, v=dv)
        hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
    torch.cuda.synchronize()
    for i, (q, k, v, out, *_rest) in enumerate(runs):
        assert_close(out.cpu().numpy(), ref_out(oracle, q, k, v, n_kv - 1, 0.125), TOL_F32, f"launch {i}")


def test_decode_qwen7b_shape_f16_cache(hip, stream, oracle, decode_mode):
    n_kv = 8192
    q, k, v = cpu_attention.make_inputs(1238, 128, 28, 4, n_kv, 1)
    scale = float(np.float32(1) / np.sqrt(np.float32(128)))
    got = fused(hip, stream, q, k, v, n_kv - 1, scale, f16=True)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale, f16=True), TOL_F32, "widened")
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale), TOL_F16, "unrounded")


def batch_24(hip, stream, n_kv, seed0, ws=None, st=None):
    """24 independent single-layer decode problems at the Qwen2.5-0.5B shape in one
    mi_hip_attn_decode_batch call; returns (inputs, device outputs)."""
    import torch
    n_layers = 24
    ins, outs, items = [], [], []
    for layer in range(n_layers):
        q, k, v = cpu_attention.make_inputs(seed0 + layer, 64, 14, 2, n_kv, 1)
        ins.append((q, k, v))
    dev_in = [(dev(q), dev(k), dev(v)) for q, k, v in ins]
    for layer in range(n_layers):
        out = torch.full((1, 14, 64), float("nan"), device="cuda")
        outs.append(out)
        dq, dk, dv = dev_in[layer]
        items.append(mh.attn_args(dq, out, 7, n_kv - 1 - layer, 0.125, st or stream, k=dk, v=dv, ws=ws))
    arr = (mh.AttnArgs * n_layers)(*items)
    hip.check(hip.mi_hip_attn_decode_batch(arr, n_layers, st or stream))
    return ins, outs, dev_in


def check_batch_24(oracle, ins, outs, n_kv, what=""):
    for layer, (q, k, v) in enumerate(ins):
        want = ref_out(oracle, q, k, v, n_kv - 1 - layer, 0.125)
        assert_close(outs[layer].cpu().numpy(), want, TOL_F32, f"{what} layer {layer}")


def test_early_merge_fallback_is_exact(hip, stream, oracle, tuning):
    # A poll limit of 0 makes every early merger stop polling at once. A merger
    # whose parts have all started keeps waiting for them; one whose group
    # straddles the set of resident workgroups (32 items x 2 groups x 8 parts =
    # 512 workgroups, about two per CU, with the early protocol forced) gives
    # up, and the last of its parts that started after that merges. Results
    # must be exact either way, and no group may be lost.
    import torch
    ws = hip.workspace_create(2, 14, 64)
    try:
        hip.check(hip.mi_hip_workspace_set_poll_limit(ws, 0))
        for rep in range(3):
            ins, outs, _ = batch_24(hip, stream, 4096, 7000 + 100 * rep, ws=ws)
            torch.cuda.synchronize()
            check_batch_24(oracle, ins, outs, 4096, f"rep {rep}")
            rc, fallbacks, lost = hip.workspace_check(ws, stream)
            print("all resident: fallbacks", fallbacks, "lost", lost, flush=True)
            assert rc == 0 and lost == 0
        tuning(kpg=8, early=2)
        hip.check(hip.mi_hip_workspace_destroy(ws))
        ws = hip.workspace_create(2, 14, 64)  # sized for the forced split
        hip.check(hip.mi_hip_workspace_set_poll_limit(ws, 0))
        total = 0
        for rep in range(4):
            n, n_kv = 32, 2048
            qs, ks, vs, outs, items, keep = [], [], [], [], [], []
            for i in range(n):
                q, k, v = cpu_attention.make_inputs(7300 + 50 * rep + i, 64, 14, 2, n_kv, 1)
                qs.append(q); ks.append(k); vs.append(v)
                dq, dk, dv = dev(q), dev(k), dev(v)
                out = torch.full((1, 14, 64), float("nan"), device="cuda")
                keep.append((dq, dk, dv)); outs.append(out)
                items.append(mh.attn_args(dq, out, 7, n_kv - 1, 0.125, stream, k=dk, v=dv, ws=ws))
            arr = (mh.AttnArgs * n)(*items)
            hip.check(hip.mi_hip_attn_decode_batch(arr, n, stream))
            torch.cuda.synchronize()
            for i in range(n):
                assert_close(outs[i].cpu().numpy(), ref_out(oracle, qs[i], ks[i], vs[i], n_kv - 1, 0.125),
                             TOL_F32, f"rep {rep} item {i}")
            rc, fallbacks, lost = hip.workspace_check(ws, stream)
            print("512 workgroups: fallbacks", fallbacks, "lost", lost, flush=True)
            assert rc == 0 and lost == 0
            total += fallbacks
        print("fallbacks over 4 launches", total, flush=True)
        tuning(kpg=0, early=1)
        hip.check(hip.mi_hip_workspace_destroy(ws))
        ws = hip.workspace_create(2, 14, 64)
        ins, outs, _ = batch_24(hip, stream, 4096, 7500, ws=ws)
        torch.cuda.synchronize()
        check_batch_24(oracle, ins, outs, 4096, "default limit")
        rc, fallbacks, lost = hip.workspace_check(ws, stream)
        assert rc == 0 and lost == 0
    finally:
        hip.check(hip.mi_hip_workspace_destroy(ws))


def test_two_workspaces_decode_concurrently(hip, oracle):
    # Two sequences' decodes on two streams with their own workspaces, issued
    # without synchronisation so that the launches overlap on the device (each
    # wants a workgroup on nearly every CU, so neither is wholly resident: the
    # early mergers' bounded waits and the fallback get exercised too).
    import torch
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    w1, w2 = hip.workspace_create(2, 14, 64), hip.workspace_create(2, 14, 64)
    try:
        runs = []
        for rep in range(4):
            for st, ws, seed in ((s1, w1, 8000), (s2, w2, 9000)):
                ins, outs, keep = batch_24(hip, None, 4096, seed + 100 * rep, ws=ws, st=st.cuda_stream)
                runs.append((ins, outs, keep))
        torch.cuda.synchronize()
        for i, (ins, outs, _) in enumerate(runs):
            check_batch_24(oracle, ins, outs, 4096, f"launch {i}")
        for st, ws in ((s1, w1), (s2, w2)):
            rc, fallbacks, lost = hip.workspace_check(ws, st.cuda_stream)
            print("fallbacks", fallbacks, flush=True)
            assert rc == 0 and lost == 0
    finally:
        torch.cuda.synchronize()
        hip.check(hip.mi_hip_workspace_destroy(w1))
        hip.check(hip.mi_hip_workspace_destroy(w2))


@pytest.mark.parametrize("det", [1, 0])
@pytest.mark.parametrize("early", [1, 0])
def test_decode_batch_24_layers(hip, stream, oracle, tuning, early, det, decode_mode):
    # both cross-workgroup combines at the headline shape (5 workgroups per
    # group): the first finisher polling stamped records, and the counters
    import torch
    tuning(early=early, det=det)
    n_layers, n_kv = 24, 4096
    qs, ks, vs, outs, items = [], [], [], [], []
    for layer in range(n_layers):
        q, k, v = cpu_attention.make_inputs(5000 + layer, 64, 14, 2, n_kv, 1)
        qs.append(q)
        ks.append(k)
        vs.append(v)
    dq = [dev(q) for q in qs]
    dk = [dev(k) for k in ks]
    dv = [dev(v) for v in vs]
    douts = [torch.full((1, 14, 64), float("nan"), device="cuda") for _ in range(n_layers)]
    for layer in range(n_layers):
        items.append(mh.attn_args(dq[layer], douts[layer], 7, n_kv - 1 - layer, 0.125, stream,
                                  k=dk[layer], v=dv[layer]))
    arr = (mh.AttnArgs * n_layers)(*items)
    hip.check(hip.mi_hip_attn_decode_batch(arr, n_layers, stream))
    torch.cuda.synchronize()
    for layer in range(n_layers):
        want = ref_out(oracle, qs[layer], ks[layer], vs[layer], n_kv - 1 - layer, 0.125)
        assert_close(douts[layer].cpu().numpy(), want, TOL_F32, f"layer {layer}")


# The 24-layer batched launch of the decode sweep at every n_kv it is timed
# at (4096 above), each layer an independent cache with its own context
# length (n_kv - layer), generated on the device. All layers are checked
# against the oracle up to n_kv 1024, a fixed sample of six beyond (the
# planner lays the launch out by its total work, so the sample's launch is
# the timed one).
@pytest.mark.parametrize("n_kv", [128, 1024, 16384, 32768])
def test_decode_batch_24_layers_sweep(hip, stream, oracle, n_kv, decode_mode):
    import torch
    print("24-layer batch n_kv", n_kv, flush=True)
    n_layers = 24
    gen = torch.Generator(device="cuda").manual_seed(7100 + n_kv)
    k = torch.randn((n_layers, n_kv, 2, 64), device="cuda", generator=gen)
    v = torch.randn((n_layers, n_kv, 2, 64), device="cuda", generator=gen)
    q = torch.randn((n_layers, 1, 14, 64), device="cuda", generator=gen)
    out = torch.full_like(q, float("nan"))
    items = (mh.AttnArgs * n_layers)(*[
        mh.attn_args(q[i], out[i], 7, n_kv - 1 - i, 0.125, stream, k=k[i], v=v[i])
        for i in range(n_layers)])
    hip.check(hip.mi_hip_attn_decode_batch(items, n_layers, stream))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    layers = range(n_layers) if n_kv <= 1024 else (0, 1, 7, 12, 18, 23)
    for i in layers:
        n = n_kv - i
        want = ref_out(oracle, q[i].cpu().numpy(), k[i, :n].cpu().numpy(), v[i, :n].cpu().numpy(),
                       n - 1, 0.125)
        assert_close(got[i], want, TOL_F32, f"layer {i} (n_kv {n})")


# Scores far from N(0,1): q and k scaled by s (score standard deviation ~s^2).
# The float-product forms (the defaults) hold the F32 bar at any magnitude;
# the split-bf16 matrix forms (~2^-16 per product) hold it up to s = 2, the
# limit their documentation states.
@pytest.mark.parametrize("s", [2.0, 4.0, 8.0])
@pytest.mark.parametrize("n_kv", [777, 4096])
def test_decode_large_scores(hip, stream, oracle, s, n_kv, decode_mode):
    if decode_mode == mh.MI_HIP_DECODE_MATRIX and s > 2.0:
        pytest.skip("split-bf16 products: documented for q, k scaled by at most 2")
    print("decode large scores", s, n_kv, decode_mode, flush=True)
    q, k, v = cpu_attention.make_inputs(6100 + n_kv + int(s), 64, 14, 2, n_kv, 1)
    q, k = (q * np.float32(s)).astype(np.float32), (k * np.float32(s)).astype(np.float32)
    got = fused(hip, stream, q, k, v, n_kv - 1, 0.125)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, 0.125), TOL_F32, f"s={s}")


@pytest.mark.parametrize("s", [2.0, 4.0, 8.0])
def test_decode_large_scores_f16_cache(hip, stream, oracle, s):
    # the default form for an F16 cache (matrix cores, f16 operands, Q and P
    # split into f16 pairs), against the oracle on the widened cache
    print("decode large scores f16", s, flush=True)
    q, k, v = cpu_attention.make_inputs(6300 + int(s), 128, 28, 4, 4096, 1)
    q, k = (q * np.float32(s)).astype(np.float32), (k * np.float32(s)).astype(np.float32)
    scale = float(np.float32(1) / np.sqrt(np.float32(128)))
    got = fused(hip, stream, q, k, v, 4095, scale, f16=True)
    assert_close(got, ref_out(oracle, q, k, v, 4095, scale, f16=True), TOL_F32, f"s={s}")


@pytest.mark.parametrize("s", [2.0, 4.0, 8.0])
@pytest.mark.parametrize("mode", [mh.MI_HIP_PREFILL_F32, mh.MI_HIP_PREFILL_SPLIT_BF16])
def test_prefill_large_scores(hip, stream, oracle, prefill_mode, mode, s):
    if mode == mh.MI_HIP_PREFILL_SPLIT_BF16 and s > 2.0:
        pytest.skip("split-bf16 products: documented for q, k scaled by at most 2")
    print("prefill large scores", s, mode, flush=True)
    prefill_mode(mode)
    q, k, v = cpu_attention.make_inputs(6200 + int(s), 64, 14, 2, 300, 300)
    q, k = (q * np.float32(s)).astype(np.float32), (k * np.float32(s)).astype(np.float32)
    got = fused(hip, stream, q, k, v, 0, 0.125)
    assert_close(got, ref_out(oracle, q, k, v, 0, 0.125), TOL_F32, f"s={s}")


@pytest.mark.parametrize("n_past,n_tok,d,h,hkv", [
    (0, 1024, 64, 14, 2),     # the prefill-1024 config, full oracle
    (0, 33, 64, 14, 2),
    (37, 100, 64, 14, 2),     # chunked prefill, n_past not a multiple of 32
    (64, 96, 64, 4, 2),
    (5, 200, 128, 8, 2),
    (0, 500, 128, 28, 4),
    (300, 2, 64, 14, 2),
])
@pytest.mark.parametrize("mode", [mh.MI_HIP_PREFILL_SPLIT_BF16, mh.MI_HIP_PREFILL_F32])
def test_prefill_vs_oracle(hip, stream, oracle, prefill_mode, mode, n_past, n_tok, d, h, hkv):
    print("prefill", n_past, n_tok, d, h, hkv, mode, flush=True)
    prefill_mode(mode)
    q, k, v = cpu_attention.make_inputs(777 + n_tok, d, h, hkv, n_past + n_tok + 3, n_tok)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_past, scale)
    assert_close(got, ref_out(oracle, q, k, v, n_past, scale), TOL_F32)


@pytest.mark.parametrize("n_past,n_tok,d,f16", [
    (0, 45, 64, False), (37, 100, 64, False), (5, 200, 128, False), (11, 70, 128, True),
    (70, 1, 64, False), (99, 1, 128, True),
])
def test_cache_rows_past_n_kv_are_never_used(hip, stream, oracle, n_past, n_tok, d, f16):
    # The cache holds more rows than n_kv = n_past + n_tok and those rows are
    # NaN: a kernel that read them into a sum (even with weight 0) would
    # return NaN. The last key tile crosses n_kv in every case.
    print("rows past n_kv", n_past, n_tok, d, f16, flush=True)
    n_kv = n_past + n_tok
    q, k, v = cpu_attention.make_inputs(31 * n_kv + d, d, 14, 2, n_kv + 40, n_tok)
    k[n_kv:] = np.nan
    v[n_kv:] = np.nan
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_past, scale, f16)
    want = ref_out(oracle, q, k[:n_kv], v[:n_kv], n_past, scale, f16)
    assert_close(got, want, TOL_F32, f"n_past={n_past} n_tok={n_tok} d={d} f16={f16}")


def test_prefill_f16_cache(hip, stream, oracle):
    q, k, v = cpu_attention.make_inputs(4242, 64, 14, 2, 300, 257)
    got = fused(hip, stream, q, k, v, 43, 0.125, f16=True)
    assert_close(got, ref_out(oracle, q, k, v, 43, 0.125, f16=True), TOL_F32)


# An F16 cache in every product mode: float products on the FP32 matrix
# cores, or (the split mode, and the default for an F16 cache) f16 products,
# exact in the cache operand, with Q and P as f16 pairs (~2^-22 per product),
# at any score magnitude; queries beyond 2^14 in magnitude are scaled by a
# power of two that the scores undo.
@pytest.mark.parametrize("n_past,n_tok,d,h,hkv", [
    (0, 1024, 64, 14, 2), (37, 100, 64, 14, 2), (0, 500, 128, 28, 4), (5, 200, 128, 8, 2), (300, 2, 64, 14, 2),
])
@pytest.mark.parametrize("mode", [mh.MI_HIP_PREFILL_AUTO, mh.MI_HIP_PREFILL_SPLIT_BF16, mh.MI_HIP_PREFILL_F32])
def test_prefill_f16_cache_vs_oracle(hip, stream, oracle, prefill_mode, mode, n_past, n_tok, d, h, hkv):
    print("prefill f16", n_past, n_tok, d, h, hkv, mode, flush=True)
    prefill_mode(mode)
    q, k, v = cpu_attention.make_inputs(5777 + n_tok + d, d, h, hkv, n_past + n_tok + 3, n_tok)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_past, scale, f16=True)
    assert_close(got, ref_out(oracle, q, k, v, n_past, scale, f16=True), TOL_F32)


@pytest.mark.parametrize("s", [2.0, 4.0])
@pytest.mark.parametrize("mode", [mh.MI_HIP_PREFILL_SPLIT_BF16, mh.MI_HIP_PREFILL_F32])
def test_prefill_f16_cache_large_scores(hip, stream, oracle, prefill_mode, mode, s):
    # q and k scaled by s (score standard deviation ~s^2 over N(0,1) inputs)
    print("prefill f16 large scores", s, mode, flush=True)
    prefill_mode(mode)
    q, k, v = cpu_attention.make_inputs(6400 + int(s), 64, 14, 2, 300, 300)
    q, k = (q * np.float32(s)).astype(np.float32), (k * np.float32(s)).astype(np.float32)
    got = fused(hip, stream, q, k, v, 0, 0.125, f16=True)
    assert_close(got, ref_out(oracle, q, k, v, 0, 0.125, f16=True), TOL_F32, f"s={s}")


@pytest.mark.parametrize("mode", [mh.MI_HIP_PREFILL_SPLIT_BF16, mh.MI_HIP_PREFILL_F32])
def test_prefill_f16_cache_large_queries(hip, stream, oracle, prefill_mode, mode):
    # Queries far outside the f16 range on some heads (|q| up to ~4e5), the
    # others unscaled: the split mode's f16 query pairs are scaled by a power
    # of two that the scores undo, and the result must not change.
    print("prefill f16 large queries", mode, flush=True)
    prefill_mode(mode)
    n_past, n_tok, d = 40, 200, 128
    q, k, v = cpu_attention.make_inputs(4343, d, 8, 2, n_past + n_tok, n_tok)
    q = q.copy()
    q[:, 1] *= 1e5
    q[:, 6] *= 3e4
    q[:, 7] *= 50.0
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    got = fused(hip, stream, q, k, v, n_past, scale, f16=True)
    assert np.isfinite(got).all()
    assert_close(got, ref_out(oracle, q, k, v, n_past, scale, f16=True), TOL_F32, "widened")


def test_prefill_4096_rows_equal_decode_oracle(hip, stream, oracle):
    # Size-independent property at the full n=4096: causal row j of a prefill
    # is exactly a decode at n_past = j, which the oracle runs in O(n).
    n = 4096
    q, k, v = cpu_attention.make_inputs(1237 + 4096, 64, 14, 2, n, n)
    got = fused(hip, stream, q, k, v, 0, 0.125)
    for j in (0, 1, 31, 32, 33, 511, 1000, 2047, 3000, 4064, 4095):
        want = oracle.attention(q[j:j + 1], k, v, j, 0.125, 8)[2]
        assert_close(got[j:j + 1], want, TOL_F32, f"row {j}")


def test_kv_cache_write_and_attend(hip, stream, oracle, golden_manifest):
    import torch
    for name in ("c1_decode", "prefill_chunked", "c4_f16_decode", "d128_prefill"):
        c = golden_manifest["cases"][name]
        q, k, v = case_inputs(c)
        f16 = c["kv_type"] == "f16"
        kv = hip.kv_create(2, c["n_ctx"], c["n_head_kv"], c["head_dim"], c["n_head"],
                           mh.MI_TYPE_F16 if f16 else mh.MI_TYPE_F32)
        try:
            n_kv = c["n_past"] + c["n_tokens"]
            nb = (ctypes.c_size_t * 3)(4, 4 * c["head_dim"], 4 * c["head_dim"] * c["n_head_kv"])
            # K from the host in two pieces, V from the device in one.
            kk = np.ascontiguousarray(k[:n_kv])
            half = n_kv // 2
            hip.check(hip.mi_hip_kv_write(kv, 1, 0, 0, half, kk.ctypes.data, nb, 0, None))
            hip.check(hip.mi_hip_kv_write(kv, 1, 0, half, n_kv - half, kk[half:].ctypes.data,
                                          nb, 0, None))
            dvv = dev(v[:n_kv])
            hip.check(hip.mi_hip_kv_write(kv, 1, 1, 0, n_kv, dvv.data_ptr(), nb, 1, stream))
            dq = dev(q)
            out = torch.full(q.shape, float("nan"), device="cuda")
            a = mh.attn_args(dq, out, c["n_head"] // c["n_head_kv"], c["n_past"], c["scale"],
                             stream, kv=kv, layer=1)
            hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
            torch.cuda.synchronize()
            assert_close(out.cpu().numpy(), load_golden(name)["out"], TOL_F32, name)
            # The cache holds exactly the rounded rows in the engine layout.
            ptr, ne, nbv = hip.kv_view(kv, 1, 0)
            assert ne[:3] == [c["head_dim"], c["n_head_kv"], c["n_ctx"]]
            assert nbv[0] == (2 if f16 else 4)
            # Out-of-range requests fail cleanly.
            a.n_past = c["n_ctx"]
            assert hip.mi_hip_attn_fwd(ctypes.byref(a)) == 1
            a.n_past, a.layer = c["n_past"], 2
            assert hip.mi_hip_attn_fwd(ctypes.byref(a)) == 1
            assert hip.mi_hip_kv_write(kv, 0, 0, c["n_ctx"], 1, kk.ctypes.data, nb, 0, None) == 1
        finally:
            hip.check(hip.mi_hip_kv_destroy(kv))


@pytest.fixture()
def prefill_mode(hip):
    """Sets the prefill kernel's matrix-core mode for one test; the default afterwards."""
    def set_(mode):
        hip.check(hip.mi_hip_set_prefill_mode(mode))
    yield set_
    hip.check(hip.mi_hip_set_prefill_mode(mh.MI_HIP_PREFILL_AUTO))


@pytest.mark.parametrize("mode", [mh.MI_HIP_PREFILL_F32, mh.MI_HIP_PREFILL_SPLIT_BF16])
def test_prefill_then_decode_equals_one_prefill(hip, stream, prefill_mode, mode):
    # The engine's batch-vs-incremental check (tests/test_model_qwen2.cpp:87-134)
    # restated for the attention path: one prefill of T tokens equals a
    # prefill of the first P followed by T - P single-token decodes. With
    # float products in both kernels they agree to 2e-6; with the prefill's
    # bf16-pair products (~1e-5 relative per product) to the parity bar.
    import torch
    prefill_mode(mode)
    T, P = 70, 50
    q, k, v = cpu_attention.make_inputs(8080, 64, 14, 2, 128, T)
    kv = hip.kv_create(1, 128, 2, 64, 14)
    try:
        nb = (ctypes.c_size_t * 3)(4, 256, 512)
        hip.check(hip.mi_hip_kv_write(kv, 0, 0, 0, T, np.ascontiguousarray(k[:T]).ctypes.data, nb, 0, None))
        hip.check(hip.mi_hip_kv_write(kv, 0, 1, 0, T, np.ascontiguousarray(v[:T]).ctypes.data, nb, 0, None))
        dq = dev(q)
        whole = torch.zeros((T, 14, 64), device="cuda")
        a = mh.attn_args(dq, whole, 7, 0, 0.125, stream, kv=kv, layer=0)
        hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
        parts = torch.zeros((T, 14, 64), device="cuda")
        a = mh.attn_args(dq[:P], parts[:P], 7, 0, 0.125, stream, kv=kv, layer=0)
        hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
        for j in range(P, T):
            a = mh.attn_args(dq[j:j + 1], parts[j:j + 1], 7, j, 0.125, stream, kv=kv, layer=0)
            hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
        torch.cuda.synchronize()
        tol = dict(atol=2e-6, rtol=2e-6) if mode == mh.MI_HIP_PREFILL_F32 else TOL_F32
        assert_close(parts.cpu().numpy(), whole.cpu().numpy(), tol)
    finally:
        hip.check(hip.mi_hip_kv_destroy(kv))
