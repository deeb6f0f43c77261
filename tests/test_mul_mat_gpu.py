"""GPU Q8_0 activation quantization and Q8_0-weight matrix products.

Bar: bit-exact. The activation quantizer uses correctly rounded division and
round-half-to-even like the engine; the dot product keeps the eight float
accumulators, the fused multiply-adds and the horizontal-sum order of the
reference's default (AVX2 + FMA) path, with exact int8 byte-group sums. Checked
against the reference's own outputs (tests/golden/q8_*.npz) and, at full model
shapes, against the oracle (which equals the reference bitwise on the goldens).
"""
import ctypes

import numpy as np
import pytest

from conftest import load_golden
from oracle import cpu_attention
import mi_hip_attn as mh
from mi_hip_attn import make_tensor

pytestmark = pytest.mark.gpu


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def q8_weights(rng, n, k, w_nb1=None):
    """Random Q8_0 weight rows (raw bytes) with a row stride of w_nb1 bytes."""
    row = k // 32 * 34
    w_nb1 = w_nb1 or row
    scales = (np.abs(rng.standard_normal((n, k // 32))) * 0.002 + 1e-4).astype(np.float16)
    qs = rng.integers(-127, 128, size=(n, k // 32, 32), dtype=np.int8)
    blocks = np.empty((n, k // 32, 34), np.uint8)
    blocks[:, :, :2] = scales.view(np.uint8).reshape(n, k // 32, 2)
    blocks[:, :, 2:] = qs.view(np.uint8)
    out = np.zeros((n, w_nb1), np.uint8)
    out[:, :row] = blocks.reshape(n, row)
    return out


def quantize_on_device(hip, stream, x, act_nb1=None):
    """F32 rows x (m, k) -> device Q8_0_ACT tensor (m columns of act_nb1 bytes)."""
    import torch
    m, k = x.shape
    act_nb1 = act_nb1 or k // 32 * 36
    dx = dev(x)
    act = torch.zeros(m * act_nb1, dtype=torch.uint8, device="cuda")
    s = make_tensor(dx.data_ptr(), [k, m], [4, 4 * k])
    q = make_tensor(act.data_ptr(), [k, m], [36, act_nb1], type_=mh.MI_TYPE_Q8_0_ACT,
                    op=mh.MI_OP_QUANTIZE_Q8_0, src=[s])
    hip.check(hip.mi_hip_op_quantize_q8_0(ctypes.byref(q), stream))
    return dx, act, q


def mul_mat_on_device(hip, stream, w_raw, k, n, act, q, m, dst_nb1=None):
    import torch
    dw = dev(w_raw)
    dst_nb1 = dst_nb1 or 4 * n
    out = torch.full((m * dst_nb1 // 4,), float("nan"), device="cuda")
    wt = make_tensor(dw.data_ptr(), [k, n], [34, w_raw.shape[1]], type_=mh.MI_TYPE_Q8_0)
    d = make_tensor(out.data_ptr(), [n, m], [4, dst_nb1], op=mh.MI_OP_MUL_MAT, src=[wt, q])
    hip.check(hip.mi_hip_op_mul_mat(ctypes.byref(d), stream))
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(m, dst_nb1 // 4)[:, :n], dw


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_q8_0_reproduces_reference_goldens(hip, stream, golden_manifest):
    import torch
    for name, c in golden_manifest["q8_0"].items():
        g = load_golden(name)
        k, n, m = c["k"], c["n"], c["m"]
        _, act, q = quantize_on_device(hip, stream, g["x"])
        torch.cuda.synchronize()
        assert np.array_equal(act.cpu().numpy(), g["act"]), name
        got, _ = mul_mat_on_device(hip, stream, g["w"].reshape(n, k // 32 * 34), k, n, act, q, m)
        assert np.array_equal(bits(got), bits(g["dst"])), name


@pytest.mark.parametrize("k,n,m", [
    (896, 896, 1),      # Qwen2.5-0.5B attention output projection, one token
    (896, 896, 7),
    (896, 4864, 1),     # ffn_gate / ffn_up
    (4864, 896, 2),     # ffn_down
    (896, 131, 13),     # rows not a multiple of 32, two column chunks
    (3584, 512, 1),     # Qwen2.5-7B hidden size
    (896, 1152, 128),   # a 128-token prompt through the stacked Q/K/V rows
    (96, 9, 2),         # odd block count: 102-byte rows end mid-dword (staged form)
    (4832, 75, 1),      # 151 blocks per row, a 3-row last group
])
def test_q8_0_model_shapes_equal_oracle(hip, stream, oracle, k, n, m):
    rng = np.random.default_rng(k + n + m)
    w = q8_weights(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    _, act, q = quantize_on_device(hip, stream, x)
    got, _ = mul_mat_on_device(hip, stream, w, k, n, act, q, m)
    want_act = oracle.quantize_q8_0_act(x)
    assert np.array_equal(act.cpu().numpy(), want_act)
    want = oracle.mul_mat_q8_0(w, want_act, k, n, m)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("k,n,m", [(896, 100, 3), (4864, 61, 3)])
def test_q8_0_strided_operands(hip, stream, oracle, k, n, m):
    # padded weight rows, padded activation columns, a destination column
    # stride wider than n: only the owned bytes are read or written (the
    # second shape takes the LDS-staged form, whose last group ends at its
    # last row's last block, not at the padded stride)
    import torch
    rng = np.random.default_rng(77)
    w = q8_weights(rng, n, k, w_nb1=k // 32 * 34 + 6)
    x = rng.standard_normal((m, k)).astype(np.float32)
    act_nb1 = k // 32 * 36 + 8
    _, act, q = quantize_on_device(hip, stream, x, act_nb1=act_nb1)
    got, _ = mul_mat_on_device(hip, stream, w, k, n, act, q, m, dst_nb1=4 * (n + 5))
    a = act.cpu().numpy().reshape(m, act_nb1)
    assert not a[:, k // 32 * 36:].any()  # the column padding stayed zero
    want_act = oracle.quantize_q8_0_act(x)
    assert np.array_equal(np.ascontiguousarray(a[:, :k // 32 * 36]).reshape(-1), want_act)
    want = oracle.mul_mat_q8_0(np.ascontiguousarray(w[:, :k // 32 * 34]), want_act, k, n, m)
    assert np.array_equal(bits(got), bits(want))
