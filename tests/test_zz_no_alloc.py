"""The allocation-free decode entry point (mi_hip_attn_decode_batch_noalloc)
against the regular one (mi_hip_attn_decode_batch) on the same inputs.

Bar: |noalloc - regular| <= 1e-4 + 1e-4*|regular| (the F32 parity bar; the
fused kernels' accumulation order follows which wave takes which sub-tile, so
two launches agree to rounding, not bitwise). Two calls in a row, the second
smaller, share the scratch; neither may allocate device memory, and a launch
beyond the scratch's capacity is refused before anything runs. The scratch
keeps its contents across mi_hip_shutdown / mi_hip_init, and so does the
stamp sequence over it: a call after a new init is checked against the
oracle. Launches under graph capture are refused (a captured launch would
replay its stamp).
"""
import ctypes

import numpy as np
import pytest

from conftest import TOL_F32
from oracle import cpu_attention
import mi_hip_attn as mh

pytestmark = pytest.mark.gpu


def _items(n_items, n_kv, seed, h=14, hkv=2, d=64):
    import torch
    gen = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn((n_items, n_kv, hkv, d), device="cuda", generator=gen)
    v = torch.randn((n_items, n_kv, hkv, d), device="cuda", generator=gen)
    q = torch.randn((n_items, 1, h, d), device="cuda", generator=gen)
    return q, k, v


def _run(hip, fn, q, k, v, n_kv, stream):
    import torch
    n = q.shape[0]
    h, hkv, d = q.shape[2], k.shape[2], q.shape[3]
    out = torch.full_like(q, float("nan"))
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    items = (mh.AttnArgs * n)(*[mh.attn_args(q[i], out[i], h // hkv, n_kv - 1 - i, scale, stream,
                                             k=k[i], v=v[i]) for i in range(n)])
    rc = fn(items, n, stream)
    return rc, out


def _close(got, want, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = TOL_F32["atol"] + TOL_F32["rtol"] * np.abs(want.astype(np.float64))
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert np.all(err <= bound), f"{what}: max abs err {err.max():.3e}"


def test_noalloc_matches_regular_entry_point(hip, stream):
    import torch
    before = hip.alloc_stats()
    cases = [(24, 4096, 11), (5, 700, 12)]  # the second call is smaller
    for n_items, n_kv, seed in cases:
        print("noalloc", n_items, "items at n_kv", n_kv, flush=True)
        q, k, v = _items(n_items, n_kv, seed)
        torch.cuda.synchronize()
        a0 = hip.alloc_stats()
        rc, got = _run(hip, hip.mi_hip_attn_decode_batch_noalloc, q, k, v, n_kv, stream)
        hip.check(rc)
        torch.cuda.synchronize()
        a1 = hip.alloc_stats()
        assert (a1.n_malloc, a1.n_free, a1.bytes_live) == (a0.n_malloc, a0.n_free, a0.bytes_live)
        rc, want = _run(hip, hip.mi_hip_attn_decode_batch, q, k, v, n_kv, stream)
        hip.check(rc)
        torch.cuda.synchronize()
        _close(got.cpu().numpy(), want.cpu().numpy(), f"{n_items} items, n_kv {n_kv}")
    # one item also against the oracle (the regular path is itself pinned there)
    q, k, v = _items(1, 333, 13)
    rc, got = _run(hip, hip.mi_hip_attn_decode_batch_noalloc, q, k, v, 333, stream)
    hip.check(rc)
    torch.cuda.synchronize()
    want = cpu_attention.oracle().attention(q[0].cpu().numpy(), k[0].cpu().numpy(),
                                            v[0].cpu().numpy(), 332, 0.125, 8)[2]
    _close(got[0].cpu().numpy(), want, "oracle")
    after = hip.alloc_stats()
    assert (after.n_malloc, after.n_free) == (before.n_malloc, before.n_free)


def test_noalloc_refuses_launches_beyond_its_scratch(hip, stream):
    # 32 items x 8 KV heads = 256 groups, more than the scratch's 128: refused on
    # the host (nothing launched), and the regular entry point still works.
    import torch
    q, k, v = _items(32, 64, 14, h=16, hkv=8, d=64)
    torch.cuda.synchronize()
    rc, _ = _run(hip, hip.mi_hip_attn_decode_batch_noalloc, q, k, v, 64, stream)
    assert rc == 5, (rc, hip.last_error())  # MI_HIP_E_UNSUPPORTED
    assert "exceeds its workspace" in hip.last_error()
    rc, out = _run(hip, hip.mi_hip_attn_decode_batch, q, k, v, 64, stream)
    hip.check(rc)
    torch.cuda.synchronize()
    assert np.all(np.isfinite(out.cpu().numpy()))


def test_noalloc_after_shutdown_and_init(hip, stream):
    # records and counters from the calls above stay in the static array; the
    # session after a shutdown / init continues the stamps over them
    import torch
    q, k, v = _items(24, 4096, 15)
    rc, first = _run(hip, hip.mi_hip_attn_decode_batch_noalloc, q, k, v, 4096, stream)
    hip.check(rc)
    torch.cuda.synchronize()
    hip.check(hip.mi_hip_shutdown())
    hip.check(hip.mi_hip_init(0))
    for seed in (16, 17):
        q, k, v = _items(24, 4096, seed)
        rc, got = _run(hip, hip.mi_hip_attn_decode_batch_noalloc, q, k, v, 4096, stream)
        hip.check(rc)
        torch.cuda.synchronize()
        g = got.cpu().numpy()
        for i in (0, 11, 23):
            want = cpu_attention.oracle().attention(q[i].cpu().numpy(), k[i, :4096 - i].cpu().numpy(),
                                                    v[i, :4096 - i].cpu().numpy(), 4095 - i, 0.125, 8)[2]
            _close(g[i], want, f"after init, seed {seed}, item {i}")


def test_decode_refused_under_graph_capture(hip):
    import torch
    q, k, v = _items(2, 256, 18)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g, stream=side, capture_error_mode="thread_local"):
        st = torch.cuda.current_stream().cuda_stream
        for fn in (hip.mi_hip_attn_decode_batch_noalloc, hip.mi_hip_attn_decode_batch):
            rc, _ = _run(hip, fn, q, k, v, 256, st)
            rcs.append((rc, hip.last_error()))
    assert all(rc == 5 and "captured" in msg for rc, msg in rcs), rcs
