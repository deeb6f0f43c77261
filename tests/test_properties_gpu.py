"""Size-independent properties of the fused decode and prefill kernels, at the
workloads' full sizes, checked against what the mathematics fixes rather than
against the oracle:

- linearity in V: O(V1 + V2) = O(V1) + O(V2) (the probabilities depend on Q
  and K only);
- equal keys: every position gets the same probability, so O is the mean of
  the V rows (computed here in float64);
- a key shift K + u (one vector u for every position of a KV head) adds q.u to
  every score of a query and leaves its softmax unchanged;
- the positions are a set: permuting K and V rows together leaves O unchanged;
- causality: prefill rows before position m read nothing at or after m, so
  changing K/V there leaves those rows bit for bit the same.

Bar for the rounding-level comparisons: |got - want| <= 1e-4 + 1e-4*|want|
(F32 K/V), the bar of the oracle comparisons.
"""
import numpy as np
import pytest

from conftest import TOL_F32
from test_attn_gpu import assert_close, fused
import mi_hip_attn as mh

pytestmark = pytest.mark.gpu

H, HKV, D = 14, 2, 64
SCALE = D ** -0.5


@pytest.fixture(params=[mh.MI_HIP_DECODE_MATRIX, mh.MI_HIP_DECODE_VALU, mh.MI_HIP_DECODE_STREAM],
                ids=["matrix", "valu", "stream"])
def kernel(request, hip):
    hip.check(hip.mi_hip_set_decode_mode(request.param))
    yield request.param
    hip.check(hip.mi_hip_set_decode_mode(mh.MI_HIP_DECODE_AUTO))


def randn(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32)


@pytest.mark.parametrize("n_kv", [4096, 32768])
def test_decode_linear_in_values(hip, stream, kernel, n_kv):
    print("linearity", kernel, n_kv, flush=True)
    rng = np.random.default_rng(11 + n_kv)
    q, k = randn(rng, 1, H, D), randn(rng, n_kv, HKV, D)
    v1, v2 = randn(rng, n_kv, HKV, D), randn(rng, n_kv, HKV, D)
    o1 = fused(hip, stream, q, k, v1, n_kv - 1, SCALE)
    o2 = fused(hip, stream, q, k, v2, n_kv - 1, SCALE)
    o12 = fused(hip, stream, q, k, v1 + v2, n_kv - 1, SCALE)
    assert_close(o12, (o1.astype(np.float64) + o2), TOL_F32, "O(V1 + V2) vs O(V1) + O(V2)")


@pytest.mark.parametrize("n_kv", [1, 17, 4096, 32768])
def test_decode_equal_keys_give_the_mean_of_values(hip, stream, kernel, n_kv):
    print("equal keys", kernel, n_kv, flush=True)
    rng = np.random.default_rng(23 + n_kv)
    q = randn(rng, 1, H, D)
    k = np.broadcast_to(randn(rng, 1, HKV, D), (n_kv, HKV, D)).copy()
    v = randn(rng, n_kv, HKV, D)
    got = fused(hip, stream, q, k, v, n_kv - 1, SCALE)
    mean = v.astype(np.float64).mean(axis=0)  # [HKV, D]
    want = np.repeat(mean, H // HKV, axis=0)[None]  # head h reads KV head h // n_rep
    assert_close(got, want, TOL_F32, "equal keys vs mean of V")


@pytest.mark.parametrize("n_kv", [777, 4096])
def test_decode_key_shift_invariance(hip, stream, kernel, n_kv):
    print("key shift", kernel, n_kv, flush=True)
    rng = np.random.default_rng(31 + n_kv)
    q, k, v = randn(rng, 1, H, D), randn(rng, n_kv, HKV, D), randn(rng, n_kv, HKV, D)
    u = randn(rng, 1, HKV, D)
    got = fused(hip, stream, q, k + u, v, n_kv - 1, SCALE)
    want = fused(hip, stream, q, k, v, n_kv - 1, SCALE)
    assert_close(got, want, TOL_F32, "K + u vs K")


@pytest.mark.parametrize("n_kv", [1000, 4096])
def test_decode_position_permutation(hip, stream, kernel, n_kv):
    print("permutation", kernel, n_kv, flush=True)
    rng = np.random.default_rng(43 + n_kv)
    q, k, v = randn(rng, 1, H, D), randn(rng, n_kv, HKV, D), randn(rng, n_kv, HKV, D)
    perm = rng.permutation(n_kv)
    got = fused(hip, stream, q, k[perm], v[perm], n_kv - 1, SCALE)
    want = fused(hip, stream, q, k, v, n_kv - 1, SCALE)
    assert_close(got, want, TOL_F32, "permuted positions vs original")


@pytest.fixture(params=[mh.MI_HIP_PREFILL_SPLIT_BF16, mh.MI_HIP_PREFILL_F32], ids=["split_bf16", "f32"])
def prefill_products(request, hip):
    hip.check(hip.mi_hip_set_prefill_mode(request.param))
    yield request.param
    hip.check(hip.mi_hip_set_prefill_mode(mh.MI_HIP_PREFILL_AUTO))


@pytest.mark.parametrize("n,m", [(1024, 1000), (4096, 2049)])
def test_prefill_rows_before_m_ignore_positions_from_m(hip, stream, prefill_products, n, m):
    print("prefill causality", prefill_products, n, m, flush=True)
    rng = np.random.default_rng(53 + n)
    q, k, v = randn(rng, n, H, D), randn(rng, n, HKV, D), randn(rng, n, HKV, D)
    k2, v2 = k.copy(), v.copy()
    k2[m:] = randn(rng, n - m, HKV, D) * 3.0
    v2[m:] = randn(rng, n - m, HKV, D) * 3.0
    a = fused(hip, stream, q, k, v, 0, SCALE)
    b = fused(hip, stream, q, k2, v2, 0, SCALE)
    assert np.array_equal(a[:m].view(np.uint32), b[:m].view(np.uint32)), "rows before m changed"
    assert not np.array_equal(a[m:], b[m:]), "rows from m should see the new positions"


def test_prefill_linear_in_values(hip, stream, prefill_products):
    n = 1024
    print("prefill linearity", prefill_products, n, flush=True)
    rng = np.random.default_rng(61)
    q, k = randn(rng, n, H, D), randn(rng, n, HKV, D)
    v1, v2 = randn(rng, n, HKV, D), randn(rng, n, HKV, D)
    o1 = fused(hip, stream, q, k, v1, 0, SCALE)
    o2 = fused(hip, stream, q, k, v2, 0, SCALE)
    o12 = fused(hip, stream, q, k, v1 + v2, 0, SCALE)
    assert_close(o12, (o1.astype(np.float64) + o2), TOL_F32, "O(V1 + V2) vs O(V1) + O(V2)")


# The longest contexts one KV head's 32-bit byte offsets address: head_dim
# 64, 2 KV heads interleaved (512 bytes per position with an F32 cache, 256
# with F16). Decode: n_kv = 2^22 (F32) or 2^23 (F16), the last row ending
# 256 (128) bytes below 2^31. Prefill: 33 positions fewer (its key tiles reach
# 32 rows past n_kv). Every key is zero except one per KV
# head, aligned with every query so that its score is 40: weight e^40 against
# fewer than 2^22 < e^15.3 for all the rest, so every head's output is that
# position's V row (relative error below e^-24). Decode puts them at the very
# last position (KV head 0) and in the middle (KV head 1); prefill at the last
# cached position and in the middle, which all its queries see. One position
# more is refused before anything runs (the buffers hold 64 rows more, so no
# access could leave them either way).
N_DECODE_MAX = {"f32": 1 << 22, "f16": 1 << 23}
N_PREFILL_MAX = {"f32": (1 << 22) - 33, "f16": (1 << 23) - 33}


def _dominant_keys(torch, n_rows, stars, seed, f16):
    # (5.0 and the V rows are exact in the cache type; want is their float value)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    dt = torch.float16 if f16 else torch.float32
    k = torch.zeros((n_rows, HKV, D), device="cuda", dtype=dt)
    v = torch.randn((n_rows, HKV, D), device="cuda", generator=gen).to(dt)
    for g, pos in enumerate(stars):
        k[pos, g] = 40.0 / (SCALE * D)
    want = np.stack([v[stars[h // (H // HKV)], h // (H // HKV)].float().cpu().numpy() for h in range(H)])
    return k, v, want


@pytest.mark.parametrize("cache", ["f32", "f16"])
def test_decode_longest_context(hip, stream, kernel, cache):
    import ctypes
    import torch
    n_max = N_DECODE_MAX[cache]
    print("longest decode context", kernel, cache, n_max, flush=True)
    stars = (n_max - 1, n_max // 2 + 3)
    k, v, want = _dominant_keys(torch, n_max + 64, stars, 77, cache == "f16")
    q = torch.ones((1, H, D), device="cuda")
    out = torch.full_like(q, float("nan"))
    a = mh.attn_args(q, out, H // HKV, n_max - 1, SCALE, stream, k=k, v=v)
    hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want[None], TOL_F32, f"dominant keys at n_kv {n_max}")
    a = mh.attn_args(q, out, H // HKV, n_max, SCALE, stream, k=k, v=v)
    assert hip.mi_hip_attn_fwd(ctypes.byref(a)) == 5  # MI_HIP_E_UNSUPPORTED
    assert "2^31" in hip.last_error()
    del k, v
    torch.cuda.empty_cache()


@pytest.mark.parametrize("cache", ["f32", "f16"])
def test_prefill_longest_context(hip, stream, prefill_products, cache):
    import ctypes
    import torch
    n_tok = 32
    n_max = N_PREFILL_MAX[cache]
    n_past = n_max - n_tok
    print("longest prefill context", prefill_products, cache, n_max, flush=True)
    stars = (n_past - 1, n_past // 2 + 5)
    k, v, want = _dominant_keys(torch, n_max + 64, stars, 78, cache == "f16")
    q = torch.ones((n_tok, H, D), device="cuda")
    out = torch.full_like(q, float("nan"))
    a = mh.attn_args(q, out, H // HKV, n_past, SCALE, stream, k=k, v=v)
    hip.check(hip.mi_hip_attn_fwd(ctypes.byref(a)))
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), np.broadcast_to(want[None], (n_tok, H, D)), TOL_F32,
                 f"dominant keys at n_kv {n_max}")
    a = mh.attn_args(q, out, H // HKV, n_past + 1, SCALE, stream, k=k, v=v)
    assert hip.mi_hip_attn_fwd(ctypes.byref(a)) == 5  # MI_HIP_E_UNSUPPORTED
    assert "2^31" in hip.last_error()
    del k, v
    torch.cuda.empty_cache()
