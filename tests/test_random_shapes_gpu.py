"""Fused decode and prefill on seeded random problem shapes, against the oracle.

The other GPU tests pin chosen shapes and edge cases. These draw shapes from a
fixed seed over everything the fused entry points take (1-8 KV heads, 1-8 Q
heads per KV head, head_dim 64 or 128, F32 or F16 cache, context lengths
spread log-uniformly, scales around 1/sqrt(head_dim)), in the library's
default kernel choice, deterministic and not. That way the planner's
layouts (head chunks, parts per group, merge protocols) are reached in
combinations nobody picked by hand. Same bar as the fixed-shape tests:
|gpu - ref| <= 1e-4 + 1e-4 |ref|, with an F16 cache against the oracle on the
exactly widened cache.
"""
import numpy as np
import pytest

from conftest import TOL_F32
from oracle import cpu_attention
import mi_hip_attn as mh
from test_attn_gpu import assert_close, dev, fused, ref_out

pytestmark = pytest.mark.gpu


def _shape(rng):
    hkv = int(rng.choice([1, 2, 3, 4, 8]))
    n_rep = int(rng.integers(1, 9))
    d = int(rng.choice([64, 128]))
    f16 = bool(rng.integers(0, 2))
    scale = float(np.float32(rng.uniform(0.5, 2.0) / np.sqrt(d)))
    return hkv, n_rep, d, f16, scale


def _decode_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv, n_rep, d, f16, scale = _shape(rng)
        n_kv = int(np.exp(rng.uniform(0.0, np.log(9000.0))))
        out.append((i, hkv, n_rep, d, f16, scale, max(1, n_kv)))
    return out


def _prefill_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv, n_rep, d, f16, scale = _shape(rng)
        out.append((i, hkv, n_rep, d, f16, scale, int(rng.integers(0, 400)), int(rng.integers(2, 131))))
    return out


@pytest.fixture(params=[1, 0], ids=["det", "nondet"])
def det(request, hip):
    hip.check(hip.mi_hip_set_deterministic(request.param))
    yield request.param
    hip.check(hip.mi_hip_set_deterministic(1))


@pytest.mark.parametrize("case", _decode_cases(48, 20261202), ids=lambda c: f"d{c[0]}")
def test_random_decode(hip, stream, oracle, det, case):
    i, hkv, n_rep, d, f16, scale, n_kv = case
    print(f"decode case {i}: n_head_kv {hkv} n_rep {n_rep} D {d} f16 {f16} n_kv {n_kv} det {det}", flush=True)
    q, k, v = cpu_attention.make_inputs(900 + i, d, hkv * n_rep, hkv, n_kv, 1)
    got = fused(hip, stream, q, k, v, n_kv - 1, scale, f16)
    assert_close(got, ref_out(oracle, q, k, v, n_kv - 1, scale, f16), TOL_F32, f"decode case {i}")


@pytest.mark.parametrize("case", _prefill_cases(24, 20261203), ids=lambda c: f"p{c[0]}")
def test_random_prefill(hip, stream, oracle, det, case):
    i, hkv, n_rep, d, f16, scale, n_past, n_tok = case
    print(f"prefill case {i}: n_head_kv {hkv} n_rep {n_rep} D {d} f16 {f16} n_past {n_past} "
          f"n_tokens {n_tok} det {det}", flush=True)
    q, k, v = cpu_attention.make_inputs(1900 + i, d, hkv * n_rep, hkv, n_past + n_tok, n_tok)
    got = fused(hip, stream, q, k, v, n_past, scale, f16)
    assert_close(got, ref_out(oracle, q, k, v, n_past, scale, f16), TOL_F32, f"prefill case {i}")


@pytest.mark.parametrize("seed", [31, 32, 33, 34, 35, 36])
def test_random_decode_batch(hip, stream, oracle, det, seed):
    # one shape per batch, each item its own cache and context length
    import torch
    rng = np.random.default_rng(seed)
    hkv, n_rep, d, f16, scale = _shape(rng)
    n_items = int(rng.integers(2, 13))
    lens = [max(1, int(np.exp(rng.uniform(0.0, np.log(6000.0))))) for _ in range(n_items)]
    print(f"batch seed {seed}: n_head_kv {hkv} n_rep {n_rep} D {d} f16 {f16} n_kv {lens} det {det}",
          flush=True)
    host, keep, items = [], [], []
    for j, n_kv in enumerate(lens):
        q, k, v = cpu_attention.make_inputs(100 * seed + j, d, hkv * n_rep, hkv, n_kv, 1)
        dk = dev(k.astype(np.float16)) if f16 else dev(k)
        dv = dev(v.astype(np.float16)) if f16 else dev(v)
        dq = dev(q)
        out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
        keep += [dq, dk, dv, out]
        host.append((q, k, v, out))
        items.append(mh.attn_args(dq, out, n_rep, n_kv - 1, scale, stream, k=dk, v=dv))
    arr = (mh.AttnArgs * n_items)(*items)
    hip.check(hip.mi_hip_attn_decode_batch(arr, n_items, stream))
    torch.cuda.synchronize()
    for j, (q, k, v, out) in enumerate(host):
        want = ref_out(oracle, q, k, v, lens[j] - 1, scale, f16)
        assert_close(out.cpu().numpy(), want, TOL_F32, f"batch seed {seed} item {j} (n_kv {lens[j]})")
