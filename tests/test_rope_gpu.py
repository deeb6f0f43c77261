"""GPU RoPE (MI_OP_ROPE) and the fused RoPE + KV append of one layer's step.

Bar: the F32 tolerance |gpu - ref| <= 1e-4 + 1e-4*|ref|. The frequencies are
the host's powf values, exactly as the engine forms them, and the angle is one
rounded float product, so theta matches the engine bit for bit; the device's
cosine and sine (double, rounded to float) are within one float ulp of the
host's cosf/sinf, which are not correctly rounded. So the outputs agree to a
few float ulps; the test also asserts that tighter bound (8 ulps of the
row's largest magnitude). V is a plain copy (F32 bit-exact, F16 rounded to
nearest even like numpy's float16 cast).
"""
import ctypes

import numpy as np
import pytest

from conftest import TOL_F32, load_golden
from oracle import cpu_attention
import mi_hip_attn as mh
from mi_hip_attn import make_tensor

pytestmark = pytest.mark.gpu

QWEN05_BASE = 1000000.0


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def assert_close(got, want, what=""):
    got64, want64 = got.astype(np.float64), want.astype(np.float64)
    err = np.abs(got64 - want64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    bound = TOL_F32["atol"] + TOL_F32["rtol"] * np.abs(want64)
    assert np.all(err <= bound), f"{what}: max abs err {err.max():.3e}"
    # a few ulps of the row scale
    scale = np.abs(want64).max(axis=-1, keepdims=True) + 1e-30
    assert np.all(err <= 8 * np.spacing(np.float32(1)) * scale), f"{what}: {(err / scale).max():.3e}"


def rope_node(t_src, t_dst, n_past, n_dims, base):
    ne = [t_src.shape[2], t_src.shape[1], t_src.shape[0]]
    es = t_src.element_size()
    s = make_tensor(t_src.data_ptr(), ne, [t_src.stride(2) * es, t_src.stride(1) * es,
                                           t_src.stride(0) * es])
    d = make_tensor(t_dst.data_ptr(), ne, [t_dst.stride(2) * es, t_dst.stride(1) * es,
                                           t_dst.stride(0) * es],
                    op=mh.MI_OP_ROPE, src=[s], params=[n_past, n_dims, float(base)])
    return s, d


def test_rope_node_reproduces_reference_goldens(hip, stream, golden_manifest):
    import torch
    for name, c in golden_manifest["rope"].items():
        g = load_golden(name)
        src = dev(g["src"])
        out = torch.full_like(src, float("nan"))
        _, d = rope_node(src, out, c["n_past"], c["n_dims"], c["freq_base"])
        hip.check(hip.mi_hip_op_rope(ctypes.byref(d), stream))
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert_close(got, g["dst"], name)
        if c["n_dims"] < c["head_dim"]:
            assert np.array_equal(got[..., c["n_dims"]:], g["src"][..., c["n_dims"]:]), name


def test_rope_known_answers(hip, stream):
    import torch
    x = dev(np.array([[[1, 2, 3, 4]]], np.float32))
    y = torch.empty_like(x)
    _, d = rope_node(x, y, 0, 4, 10000.0)
    hip.check(hip.mi_hip_op_rope(ctypes.byref(d), stream))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), x.cpu().numpy())  # position 0: identity
    x = dev(np.array([[[1, 0]]], np.float32))
    y = torch.empty_like(x)
    _, d = rope_node(x, y, 5, 2, 10000.0)
    hip.check(hip.mi_hip_op_rope(ctypes.byref(d), stream))
    torch.cuda.synchronize()
    got = y.cpu().numpy()[0, 0]
    assert abs(got[0] - np.cos(5.0)) < 1e-6 and abs(got[1] - np.sin(5.0)) < 1e-6


@pytest.mark.parametrize("n_tok,n_past,d,n_dims", [(1, 4095, 64, 64), (40, 0, 64, 64),
                                                   (7, 32760, 128, 128), (5, 9, 64, 16)])
def test_rope_node_strided_views_and_in_place(hip, stream, oracle, n_tok, n_past, d, n_dims):
    # Q as the engine sees it: a per-head reshape of the projection output,
    # here a strided view (every head row padded by 8 floats); then in place.
    import torch
    h = 14
    rng = np.random.default_rng(n_tok + n_past + d)
    x = rng.standard_normal((n_tok, h, d)).astype(np.float32)
    want = oracle.rope(x, n_past, n_dims, QWEN05_BASE)
    padded = torch.zeros((n_tok, h, d + 8), device="cuda")
    padded[:, :, :d] = dev(x)
    src = padded[:, :, :d]
    out = torch.full((n_tok, h, d), float("nan"), device="cuda")
    _, nd = rope_node(src, out, n_past, n_dims, QWEN05_BASE)
    hip.check(hip.mi_hip_op_rope(ctypes.byref(nd), stream))
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), want, "strided")
    _, nd = rope_node(src, src, n_past, n_dims, QWEN05_BASE)  # in place
    hip.check(hip.mi_hip_op_rope(ctypes.byref(nd), stream))
    torch.cuda.synchronize()
    assert_close(src.cpu().numpy(), want, "in place")
    assert torch.all(padded[:, :, d:] == 0)  # the padding was not touched


def read_cache(kv, layer, which, hip, n_ctx, d, hkv, f16):
    ptr, ne, nb = hip.kv_view(kv, layer, which)
    host = np.empty((n_ctx, hkv, d), np.float16 if f16 else np.float32)
    hiprt = ctypes.CDLL("libamdhip64.so")
    hiprt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hiprt.hipMemcpy(host.ctypes.data, ptr, host.nbytes, 2) == 0  # device to host
    return host


@pytest.mark.parametrize("d,h,hkv,n_past,n_tok,f16", [
    (64, 14, 2, 511, 1, False),    # Qwen2.5-0.5B decode step
    (64, 14, 2, 13, 19, False),    # a prefill chunk
    (128, 28, 4, 299, 1, True),    # 7B shape, F16 cache
    (128, 28, 4, 0, 33, True),
])
def test_rope_append_matches_oracle(hip, stream, oracle, d, h, hkv, n_past, n_tok, f16):
    import torch
    rng = np.random.default_rng(d + n_past + n_tok)
    q = rng.standard_normal((n_tok, h, d)).astype(np.float32)
    k = rng.standard_normal((n_tok, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n_tok, hkv, d)).astype(np.float32)
    n_ctx = n_past + n_tok + 5
    kv = hip.kv_create(2, n_ctx, hkv, d, h, mh.MI_TYPE_F16 if f16 else mh.MI_TYPE_F32)
    try:
        dq, dk, dv = dev(q), dev(k), dev(v)
        qo = torch.full_like(dq, float("nan"))
        a = mh.rope_args(kv, 1, n_past, d, QWEN05_BASE, stream, dk, dv, q=dq, q_out=qo)
        hip.check(hip.mi_hip_rope_append(ctypes.byref(a)))
        torch.cuda.synchronize()
        assert_close(qo.cpu().numpy(), oracle.rope(q, n_past, d, QWEN05_BASE), "Q")
        kc = read_cache(kv, 1, 0, hip, n_ctx, d, hkv, f16)
        vc = read_cache(kv, 1, 1, hip, n_ctx, d, hkv, f16)
        k_rot = oracle.rope(k, n_past, d, QWEN05_BASE)
        rows = slice(n_past, n_past + n_tok)
        if f16:
            # rounding the few-ulp device value to half may land one half-ulp away
            assert np.allclose(kc[rows].astype(np.float32), k_rot, rtol=1e-3, atol=1e-3)
            assert np.array_equal(vc[rows], v.astype(np.float16))
        else:
            assert_close(kc[rows], k_rot, "K")
            assert np.array_equal(vc[rows].view(np.uint32), v.view(np.uint32))
        # nothing outside the step's rows, nor the other layer, was written
        assert not np.any(kc[:n_past]) and not np.any(kc[n_past + n_tok:])
        assert not np.any(vc[:n_past]) and not np.any(vc[n_past + n_tok:])
        assert not np.any(read_cache(kv, 0, 0, hip, n_ctx, d, hkv, f16))
        # in place on Q, no Q at all
        a = mh.rope_args(kv, 1, n_past, d, QWEN05_BASE, stream, dk, dv, q=dq)
        hip.check(hip.mi_hip_rope_append(ctypes.byref(a)))
        a = mh.rope_args(kv, 0, n_past, d, QWEN05_BASE, stream, dk, dv)
        hip.check(hip.mi_hip_rope_append(ctypes.byref(a)))
        torch.cuda.synchronize()
        assert_close(dq.cpu().numpy(), oracle.rope(q, n_past, d, QWEN05_BASE), "Q in place")
        kc0 = read_cache(kv, 0, 0, hip, n_ctx, d, hkv, f16)
        assert np.array_equal(kc0[rows], kc[rows])
        # positions past n_ctx are refused before any launch
        a.n_past = n_ctx - n_tok + 1
        assert hip.mi_hip_rope_append(ctypes.byref(a)) == 1
    finally:
        hip.check(hip.mi_hip_kv_destroy(kv))


def test_step_rope_append_then_attention_equals_oracle(hip, stream, oracle):
    # One decode step of src/model_qwen2.cpp:153-177 on device: the cache holds
    # n_past rotated keys, the step rotates Q and the new K, appends K and V,
    # then attends; the oracle runs the same engine ops on the host.
    import torch
    d, h, hkv, n_past = 64, 14, 2, 700
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, h, d)).astype(np.float32)
    k_all = rng.standard_normal((n_past + 1, hkv, d)).astype(np.float32)
    v_all = rng.standard_normal((n_past + 1, hkv, d)).astype(np.float32)
    k_rot = oracle.rope(k_all, 0, d, QWEN05_BASE)  # every key at its own position
    kv = hip.kv_create(1, 1024, hkv, d, h, mh.MI_TYPE_F32)
    try:
        nb = (ctypes.c_size_t * 3)(4, 4 * d, 4 * d * hkv)
        prev = np.ascontiguousarray(k_rot[:n_past])
        hip.check(hip.mi_hip_kv_write(kv, 0, 0, 0, n_past, prev.ctypes.data, nb, 0, None))
        prev_v = np.ascontiguousarray(v_all[:n_past])
        hip.check(hip.mi_hip_kv_write(kv, 0, 1, 0, n_past, prev_v.ctypes.data, nb, 0, None))
        dq, dk, dv = dev(q), dev(k_all[n_past:]), dev(v_all[n_past:])
        a = mh.rope_args(kv, 0, n_past, d, QWEN05_BASE, stream, dk, dv, q=dq)
        hip.check(hip.mi_hip_rope_append(ctypes.byref(a)))
        out = torch.full((1, h, d), float("nan"), device="cuda")
        at = mh.attn_args(dq, out, h // hkv, n_past, 0.125, stream, kv=kv, layer=0)
        hip.check(hip.mi_hip_attn_fwd(ctypes.byref(at)))
        torch.cuda.synchronize()
        q_rot = oracle.rope(q, n_past, d, QWEN05_BASE)
        want = oracle.attention(q_rot, k_rot, v_all, n_past, 0.125, 8)[2]
        got = out.cpu().numpy()
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= TOL_F32["atol"] + TOL_F32["rtol"] * np.abs(want)), err.max()
    finally:
        hip.check(hip.mi_hip_kv_destroy(kv))
