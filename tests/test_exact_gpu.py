"""mi_hip_attn_fwd_reference_order: the ATTN_QK -> SOFTMAX -> ATTN_KQV triple in
the reference's own operation order (src/ops_cpu.cpp:304-410), against the
oracle (the same order, the host C library's expf) BIT FOR BIT.

Rows of up to 512 keys at head_dim 64 (256 at 128) run the staged kernel (V
rows in LDS, the ordered sums read in chunks of 16 ahead of their additions);
longer rows run the unstaged kernel. Key counts cover one key, partial and
whole chunks of 16, odd and even chunk counts, the staged limit and past it,
prefill rows on both sides of it, and a row whose exponentials are all equal
but one (its one-lane sum rounds the same way step after step). 32 seeded
random shapes (1-8 KV heads, 1-8 Q heads each, decode rows and short
prefills, 1-3000 keys) cover head layouts the chosen cases do not.
"""
import ctypes

import numpy as np
import pytest

from oracle import cpu_attention
import mi_hip_attn as mh

pytestmark = pytest.mark.gpu


def _inputs(seed, n_tokens, n_kv, h, hkv, d):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_tokens, h, d), dtype=np.float32)
    k = rng.standard_normal((n_kv, hkv, d), dtype=np.float32)
    v = rng.standard_normal((n_kv, hkv, d), dtype=np.float32)
    return q, k, v


def _run(hip, stream, q, k, v, n_past, scale):
    import torch
    qd, kd, vd = (torch.from_numpy(x).cuda() for x in (q, k, v))
    out = torch.full_like(qd, float("nan"))
    a = mh.attn_args(qd, out, q.shape[1] // k.shape[1], n_past, scale, stream, k=kd, v=vd)
    hip.check(hip.mi_hip_attn_fwd_reference_order(ctypes.byref(a)))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _check(hip, stream, q, k, v, n_past, scale, what):
    print(what, flush=True)
    got = _run(hip, stream, q, k, v, n_past, scale)
    want = cpu_attention.oracle().attention(q, k, v, n_past, scale, 8)[2]
    diff = np.flatnonzero(_bits(got) != _bits(want))
    assert diff.size == 0, (f"{what}: {diff.size} of {got.size} outputs differ in their bits, first at "
                            f"{np.unravel_index(diff[0], got.shape)}: {got.flat[diff[0]]!r} vs {want.flat[diff[0]]!r}")


@pytest.mark.parametrize("d,n_kv", [(64, 1), (64, 15), (64, 16), (64, 17), (64, 33), (64, 129), (64, 256),
                                    (64, 383), (64, 512), (64, 513), (64, 1000), (128, 31), (128, 255),
                                    (128, 256), (128, 257)])
def test_decode_bit_for_bit(hip, stream, d, n_kv):
    q, k, v = _inputs(1000 + n_kv, 1, n_kv, 14, 2, d)
    _check(hip, stream, q, k, v, n_kv - 1, float(np.float32(1) / np.sqrt(np.float32(d))),
           f"decode D {d} n_kv {n_kv}")


@pytest.mark.parametrize("n_tokens,n_past,h,hkv", [(37, 100, 14, 2), (20, 600, 14, 2), (9, 0, 8, 8),
                                                    (16, 481, 28, 4)])
def test_prefill_rows_bit_for_bit(hip, stream, n_tokens, n_past, h, hkv):
    # rows of one call span staged and unstaged key counts (n_past + j + 1)
    q, k, v = _inputs(7 + n_past, n_tokens, n_past + n_tokens, h, hkv, 64)
    _check(hip, stream, q, k, v, n_past, 0.125, f"prefill {n_tokens} rows after {n_past}, {h}/{hkv} heads")


def test_equal_keys_but_one(hip, stream):
    # Every key equal but key 0: each head's exponentials are all one value but
    # one, so the one-lane sum rounds the same way step after step (its value
    # drifts far from the exact sum, which any reassociation would expose).
    n_kv, d = 512, 64
    q, k, v = _inputs(99, 1, n_kv, 14, 2, d)
    k[1:] = k[1]
    k[0] = -0.5 * k[1]
    _check(hip, stream, q, k, v, n_kv - 1, 0.125, "equal keys but one, n_kv 512")


def test_rejects_what_it_does_not_cover(hip, stream):
    import torch
    q = torch.zeros((1, 14, 64), device="cuda")
    out = torch.empty_like(q)
    k16 = torch.zeros((8, 2, 64), device="cuda", dtype=torch.float16)
    a = mh.attn_args(q, out, 7, 7, 0.125, stream, k=k16, v=k16)
    assert hip.mi_hip_attn_fwd_reference_order(ctypes.byref(a)) == 5  # MI_HIP_E_UNSUPPORTED
    assert "F32" in hip.last_error()
    k = torch.zeros((40000, 2, 64), device="cuda")
    a = mh.attn_args(q, out, 7, 39999, 0.125, stream, k=k, v=k)
    assert hip.mi_hip_attn_fwd_reference_order(ctypes.byref(a)) == 5
    assert "32768" in hip.last_error()


def _random_cases(n, seed):
    # (case, n_head_kv, n_rep, head_dim, n_past, n_tokens, scale): decode rows and
    # short prefills, key counts spread log-uniformly over 1..3000 (the staged
    # kernel below 512 keys at head_dim 64 / 256 at 128, the unstaged above)
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(rng.choice([1, 2, 3, 4, 8]))
        n_rep = int(rng.integers(1, 9))
        d = int(rng.choice([64, 128]))
        n_kv = max(1, int(np.exp(rng.uniform(0.0, np.log(3000.0)))))
        n_tok = 1 if rng.uniform() < 0.6 else int(rng.integers(2, min(n_kv, 40) + 1)) if n_kv > 1 else 1
        scale = float(np.float32(rng.uniform(0.5, 2.0) / np.sqrt(d)))
        out.append((i, hkv, n_rep, d, n_kv - n_tok, n_tok, scale))
    return out


@pytest.mark.parametrize("case", _random_cases(32, 20261204), ids=lambda c: f"r{c[0]}")
def test_random_shapes_bit_for_bit(hip, stream, case):
    i, hkv, n_rep, d, n_past, n_tok, scale = case
    q, k, v = _inputs(3000 + i, n_tok, n_past + n_tok, hkv * n_rep, hkv, d)
    _check(hip, stream, q, k, v, n_past, scale,
           f"random case {i}: n_head_kv {hkv} n_rep {n_rep} D {d} n_past {n_past} n_tokens {n_tok}")
