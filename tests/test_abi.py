"""C-ABI checks that need no GPU: the library loads, exports every symbol the
public headers declare, agrees with the engine on the mi_tensor layout
(src/tensor.h:122-160), and rejects bad arguments with status codes before it
touches a device (src: the engine's asserts become errors here)."""
import ctypes

import numpy as np
import os
import re

import pytest

import mi_hip_attn as mh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    return mh.lib()


def declared_symbols():
    names = set()
    for hdr in ("mi_hip_attn.h", "mi_hip_qwen2.h"):
        text = open(os.path.join(ROOT, "include", hdr)).read()
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(mi_hip_\w+)\(", text, re.M))
    return names


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) >= 19
    for n in names:
        assert hasattr(lib.so, n), n
    assert names == set(mh.SIGNATURES), names ^ set(mh.SIGNATURES)


def test_mi_tensor_layout_matches_engine(lib):
    lay = lib.abi_layout()
    T = mh.MiTensor
    expect = [ctypes.sizeof(T), T.type.offset, T.ne.offset, T.nb.offset, T.op.offset,
              T.op_params.offset, T.src.offset, T.data.offset, T.view_src.offset,
              T.view_offs.offset, T.n_children.offset, T.flags.offset, T.name.offset,
              T.extra.offset, ctypes.sizeof(mh.MiCgraph)]
    assert lay == expect
    # x86-64: int enum + 4 pad, ne[4] at 8, nb[4] at 40, op at 72, op_params at 76,
    # src at 112, ..., name at 160, extra at 224 -> 232 bytes; mi_cgraph 48 bytes.
    assert lay[0] == 232 and lay[3] == 40 and lay[6] == 112 and lay[13] == 224
    assert lay[14] == 48
    # ... which is what the reference's own header produces (where it was built).
    from oracle import cpu_attention
    ref = cpu_attention.reference()
    if ref is not None:
        arr = (ctypes.c_size_t * 15)()
        assert ref.lib.ref_abi_layout(arr, 15) == 0
        assert list(arr) == lay


def test_op_and_type_codes_match_engine():
    hdr = open(os.path.join(ROOT, "include", "mi_tensor.h")).read()
    codes = dict(re.findall(r"(MI_OP_\w+) = (\d+)", hdr))
    assert codes["MI_OP_SOFTMAX"] == "7" and codes["MI_OP_CPY"] == "10"
    assert codes["MI_OP_ATTN_QK"] == "16" and codes["MI_OP_ATTN_KQV"] == "17"
    assert dict(re.findall(r"(MI_TYPE_\w+) = (\d+)", hdr))["MI_TYPE_F16"] == "1"


def test_status_and_errors_without_device(lib):
    # No device work is possible here; every path below fails on its arguments
    # (or on the missing device) with a code and a message, never an abort.
    assert lib.mi_hip_attn_fwd(None) == 1 and "NULL" in lib.last_error()
    a = mh.AttnArgs()
    assert lib.mi_hip_attn_fwd(ctypes.byref(a)) == 1  # no KV source
    a.k = a.v = 16
    a.kv_type = 7
    assert lib.mi_hip_attn_fwd(ctypes.byref(a)) == 5  # unsupported type
    a.kv_type = mh.MI_TYPE_F32
    a.k_nb[:] = (4, 256, 512)
    a.v_nb[:] = (4, 256, 512)
    a.head_dim, a.n_head_kv = 80, 2
    assert lib.mi_hip_attn_fwd(ctypes.byref(a)) == 5  # head_dim 80
    a.head_dim = 64
    a.n_head, a.n_rep = 14, 6
    assert lib.mi_hip_attn_fwd(ctypes.byref(a)) == 1 and "n_rep" in lib.last_error()
    a.n_rep = 7
    a.n_past, a.n_tokens = -1, 1
    assert lib.mi_hip_attn_fwd(ctypes.byref(a)) == 1
    a.n_past, a.n_tokens = 5, 0  # no query: refused, not a silent no-op
    assert lib.mi_hip_attn_fwd(ctypes.byref(a)) == 1 and "n_tokens" in lib.last_error()
    assert lib.mi_hip_attn_decode_batch(None, 0, None) == 1
    d = mh.KvDesc(0, 16, 2, 64, 14, 0)
    h = ctypes.c_void_p()
    assert lib.mi_hip_kv_create(ctypes.byref(d), ctypes.byref(h)) == 1
    d = mh.KvDesc(2, 16, 2, 64, 13, 0)
    assert lib.mi_hip_kv_create(ctypes.byref(d), ctypes.byref(h)) == 1
    d = mh.KvDesc(2, 16, 2, 96, 14, 0)
    assert lib.mi_hip_kv_create(ctypes.byref(d), ctypes.byref(h)) == 5
    d = mh.KvDesc(2, 16, 2, 64, 14, 2)  # Q8_0 cache
    assert lib.mi_hip_kv_create(ctypes.byref(d), ctypes.byref(h)) == 5
    assert lib.mi_hip_graph_prepare(None) == 1
    t = mh.MiTensor()
    t.op = mh.MI_OP_SOFTMAX
    assert lib.mi_hip_op_attn_qk(ctypes.byref(t), None) == 1
    assert lib.mi_hip_op_attn_kqv(ctypes.byref(t), None) == 1
    assert lib.mi_hip_op_attn_fused(ctypes.byref(t), None) == 1
    # ROPE: wrong node, odd or oversized n_dims, unaligned strides, no kv
    assert lib.mi_hip_op_rope(ctypes.byref(t), None) == 1
    buf = np.zeros(64, np.float32)
    src = mh.make_tensor(buf.ctypes.data, [8, 2, 4], [4, 32, 64])
    for n_dims, code in ((7, 5), (10, 5), (-2, 5), (300, 5)):
        node = mh.make_tensor(buf.ctypes.data, [8, 2, 4], [4, 32, 64], op=mh.MI_OP_ROPE,
                              src=[src], params=[0, n_dims, 10000.0])
        assert lib.mi_hip_op_rope(ctypes.byref(node), None) == code, n_dims
    src_bad = mh.make_tensor(buf.ctypes.data, [8, 2, 4], [4, 34, 64])
    node = mh.make_tensor(buf.ctypes.data, [8, 2, 4], [4, 32, 64], op=mh.MI_OP_ROPE,
                          src=[src_bad], params=[0, 8, 10000.0])
    assert lib.mi_hip_op_rope(ctypes.byref(node), None) == 1
    assert lib.mi_hip_rope_append(None) == 1
    ra = mh.RopeArgs()
    assert lib.mi_hip_rope_append(ctypes.byref(ra)) == 1 and "NULL" in lib.last_error()
    # Q8_0: wrong nodes, F32 weights, k not a multiple of 32, unsplit rows
    t.op = mh.MI_OP_SOFTMAX
    assert lib.mi_hip_op_quantize_q8_0(ctypes.byref(t), None) == 1
    assert lib.mi_hip_op_mul_mat(ctypes.byref(t), None) == 1
    f32 = np.zeros(4096, np.float32)
    x = mh.make_tensor(f32.ctypes.data, [64, 2], [4, 256])
    q = mh.make_tensor(f32.ctypes.data, [64, 2], [36, 72], type_=mh.MI_TYPE_Q8_0_ACT,
                       op=mh.MI_OP_QUANTIZE_Q8_0, src=[x])
    x48 = mh.make_tensor(f32.ctypes.data, [48, 2], [4, 192])
    q48 = mh.make_tensor(f32.ctypes.data, [48, 2], [36, 72], type_=mh.MI_TYPE_Q8_0_ACT,
                         op=mh.MI_OP_QUANTIZE_Q8_0, src=[x48])
    assert lib.mi_hip_op_quantize_q8_0(ctypes.byref(q48), None) == 1  # 48 % 32
    xs = mh.make_tensor(f32.ctypes.data, [64, 2], [8, 512])
    qs = mh.make_tensor(f32.ctypes.data, [64, 2], [36, 72], type_=mh.MI_TYPE_Q8_0_ACT,
                        op=mh.MI_OP_QUANTIZE_Q8_0, src=[xs])
    assert lib.mi_hip_op_quantize_q8_0(ctypes.byref(qs), None) == 5  # nb[0] != 4
    wf = mh.make_tensor(f32.ctypes.data, [64, 3], [4, 256])  # F32 weights
    d = mh.make_tensor(f32.ctypes.data, [3, 2], [4, 12], op=mh.MI_OP_MUL_MAT, src=[wf, q])
    assert lib.mi_hip_op_mul_mat(ctypes.byref(d), None) == 5 and "Q8_0" in lib.last_error()
    wq = mh.make_tensor(f32.ctypes.data, [64, 3], [34, 68], type_=mh.MI_TYPE_Q8_0)
    d = mh.make_tensor(f32.ctypes.data, [3, 2], [4, 12], op=mh.MI_OP_MUL_MAT, src=[wq, x])
    assert lib.mi_hip_op_mul_mat(ctypes.byref(d), None) == 1  # activation not quantized
    d = mh.make_tensor(f32.ctypes.data, [4, 2], [4, 16], op=mh.MI_OP_MUL_MAT, src=[wq, q])
    assert lib.mi_hip_op_mul_mat(ctypes.byref(d), None) == 1  # dst rows != weight rows
    wq = mh.make_tensor(f32.ctypes.data, [64, 3], [34, 66], type_=mh.MI_TYPE_Q8_0)
    d = mh.make_tensor(f32.ctypes.data, [3, 2], [4, 12], op=mh.MI_OP_MUL_MAT, src=[wq, q])
    assert lib.mi_hip_op_mul_mat(ctypes.byref(d), None) == 1  # row stride below 2 blocks
    # A node that is not attention and not a KV write is not ours.
    t.op = 4  # ADD
    assert lib.mi_hip_compute_forward(ctypes.byref(t), 0, 1) == 0
    assert lib.mi_hip_abi_layout(None, 0) == 1


def test_init_reports_missing_device(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    rc = lib.mi_hip_init(0)
    assert rc in (2, 1) and lib.last_error()
    # Entry points that need the device refuse cleanly before init.
    d = mh.KvDesc(2, 16, 2, 64, 14, 0)
    h = ctypes.c_void_p()
    assert lib.mi_hip_kv_create(ctypes.byref(d), ctypes.byref(h)) == 6


def test_alloc_limit_and_stats(lib):
    s = lib.alloc_stats()
    assert s.n_malloc >= s.n_free
    assert lib.mi_hip_set_alloc_limit(1 << 20) == 0
    assert lib.mi_hip_set_alloc_limit(0) == 0


def test_memread_rejects_bad_arguments_without_device(lib):
    # argument checks come before any device work (addresses below are never touched)
    p, s = ctypes.c_void_p(1 << 20), ctypes.c_void_p(2 << 20)
    assert lib.mi_hip_memread(None, 256, s, 4, None) == 1 and "memread" in lib.last_error()
    assert lib.mi_hip_memread(p, 0, s, 4, None) == 1
    assert lib.mi_hip_memread(p, 250, s, 4, None) == 1
    assert lib.mi_hip_memread(ctypes.c_void_p((1 << 20) + 4), 240, s, 4, None) == 1
    assert lib.mi_hip_memread(p, 256, s, 0, None) == 1
    assert lib.mi_hip_memread(p, 256, s, 65537, None) == 1 and "n_sums" in lib.last_error()
