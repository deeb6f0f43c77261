"""GPU node-level operators and the executor hook.

- mi_hip_op_attn_qk / mi_hip_op_attn_kqv accumulate in the reference's order
  with separately rounded multiply and add, and mi_hip_op_softmax sums in key
  order with the glibc expf restated, so on the reference's own inputs they
  must reproduce the scores / probabilities / output BIT FOR BIT, on the
  reference's goldens and on 24 seeded random shapes (head_dim 4..128, F32
  and F16 caches, decode rows and short prefills) against the oracle.
- The executor hook runs a host-resident graph shaped like the engine's
  (src/model_qwen2.cpp:153-177: K/V CPY into the cache, ATTN_QK, SOFTMAX,
  ATTN_KQV) with the threading contract of src/threadpool.cpp:171-180, and
  allocates nothing in steady state (tests/test_zero_alloc.cpp's discipline).
"""
import ctypes

import numpy as np
import pytest

from conftest import TOL_F32, case_inputs, load_golden
from oracle import cpu_attention
import mi_hip_attn as mh
from mi_hip_attn import make_tensor

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def nb_of(shape_c, elt):
    """Engine nb[] for a C-contiguous numpy shape (reversed ne)."""
    ne = list(reversed(shape_c))
    nb = [elt]
    for i in range(1, len(ne)):
        nb.append(nb[-1] * ne[i - 1])
    return ne, nb


def dtensor(t, elt=4, type_=mh.MI_TYPE_F32, **kw):
    ne, nb = nb_of(tuple(t.shape), elt)
    return make_tensor(t.data_ptr(), ne, nb, type_=type_, **kw)


@pytest.mark.parametrize("name", ["c1_decode", "tiny_prefill", "tiny_decode", "prefill_chunked",
                                  "c4_f16_decode", "nrep8_decode", "mha_prefill"])
def test_node_ops_reproduce_reference(hip, stream, golden_manifest, name):
    import torch
    c = golden_manifest["cases"][name]
    g = load_golden(name)
    q, k, v = case_inputs(c)
    f16 = c["kv_type"] == "f16"
    n_kv, n_tok, n_head = c["n_past"] + c["n_tokens"], c["n_tokens"], c["n_head"]
    n_rep = n_head // c["n_head_kv"]
    dq = dev(q)
    dk = dev(k.astype(np.float16)) if f16 else dev(k)
    dv = dev(v.astype(np.float16)) if f16 else dev(v)
    kt = mh.MI_TYPE_F16 if f16 else mh.MI_TYPE_F32
    elt = 2 if f16 else 4
    tq, tk, tv = dtensor(dq), dtensor(dk, elt, kt), dtensor(dv, elt, kt)
    scores = torch.full((n_head, n_tok, n_kv), float("nan"), device="cuda")
    probs = torch.full_like(scores, float("nan"))
    out = torch.full((n_tok, n_head, c["head_dim"]), float("nan"), device="cuda")
    ts = dtensor(scores, op=mh.MI_OP_ATTN_QK, src=[tq, tk], params=[c["n_past"], n_rep])
    tp = dtensor(probs, op=mh.MI_OP_SOFTMAX, src=[ts], params=[c["n_past"], c["scale"]])
    to = dtensor(out, op=mh.MI_OP_ATTN_KQV, src=[tp, tv], params=[n_rep])
    hip.check(hip.mi_hip_op_attn_qk(ctypes.byref(ts), stream))
    hip.check(hip.mi_hip_op_softmax(ctypes.byref(tp), stream))
    torch.cuda.synchronize()
    want_s, want_p, _ = cpu_attention.oracle().attention(
        q, *( (cpu_attention.fp16_widen(k.astype(np.float16)), cpu_attention.fp16_widen(v.astype(np.float16))) if f16 else (k, v)),
        c["n_past"], c["scale"], 4)
    assert np.array_equal(bits(scores.cpu().numpy()), bits(want_s)), "scores not bit-exact"
    got_p = probs.cpu().numpy()
    assert np.array_equal(bits(got_p), bits(want_p)), \
        f"probs not bit-exact: {int((bits(got_p) != bits(want_p)).sum())} of {got_p.size} differ"
    # ATTN_KQV on the reference's own probabilities reproduces its output exactly.
    probs.copy_(torch.from_numpy(want_p))
    hip.check(hip.mi_hip_op_attn_kqv(ctypes.byref(to), stream))
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(g["out"])), "output not bit-exact"
    if c["head_dim"] in (64, 128):
        out.fill_(float("nan"))
        hip.check(hip.mi_hip_op_attn_fused(ctypes.byref(to), stream))
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.all(np.abs(got - g["out"]) <= 1e-4 + 1e-4 * np.abs(g["out"]))


def test_node_op_shape_errors(hip, stream):
    import torch
    q = torch.zeros((1, 14, 64), device="cuda")
    k = torch.zeros((16, 2, 64), device="cuda")
    s = torch.zeros((14, 1, 17), device="cuda")  # one key too many for a 16-row K
    tq, tk = dtensor(q), dtensor(k)
    ts = dtensor(s, op=mh.MI_OP_ATTN_QK, src=[tq, tk], params=[16, 7])
    assert hip.mi_hip_op_attn_qk(ctypes.byref(ts), stream) == 1
    ts = dtensor(s[:, :, :16], op=mh.MI_OP_ATTN_QK, src=[tq, tk], params=[15, 0])
    assert hip.mi_hip_op_attn_qk(ctypes.byref(ts), stream) == 1  # n_rep 0


class HostGraph:
    """The engine's per-layer attention subgraph over host buffers."""

    def __init__(self, hip, kv, layer, head_dim, n_head, n_head_kv, n_ctx):
        self.hip, self.kv, self.layer = hip, kv, layer
        self.d, self.h, self.hkv, self.n_ctx = head_dim, n_head, n_head_kv, n_ctx
        self.k_host = np.zeros((n_ctx, n_head_kv, head_dim), np.float32)
        self.v_host = np.zeros_like(self.k_host)
        ne, nb = nb_of(self.k_host.shape, 4)
        self.tk = make_tensor(self.k_host.ctypes.data, ne, nb)
        self.tv = make_tensor(self.v_host.ctypes.data, ne, nb)
        self.tk.flags = self.tv.flags = mh.MI_TENSOR_FLAG_KV
        hip.check(hip.mi_hip_kv_bind(kv, layer, 0, ctypes.byref(self.tk)))
        hip.check(hip.mi_hip_kv_bind(kv, layer, 1, ctypes.byref(self.tv)))

    def build(self, q, k_rows, v_rows, n_past, scale):
        n_tok = q.shape[0]
        n_kv = n_past + n_tok
        keep = []
        self.q, self.kr, self.vr = (np.ascontiguousarray(x) for x in (q, k_rows, v_rows))
        self.scores = np.full((self.h, n_tok, n_kv), np.nan, np.float32)
        self.probs = np.full_like(self.scores, np.nan)
        self.out = np.full((n_tok, self.h, self.d), np.nan, np.float32)
        tq = make_tensor(self.q.ctypes.data, *nb_of(self.q.shape, 4))
        tkr = make_tensor(self.kr.ctypes.data, *nb_of(self.kr.shape, 4))
        tvr = make_tensor(self.vr.ctypes.data, *nb_of(self.vr.shape, 4))
        cpys = []
        for owner, rows in ((self.tk, tkr), (self.tv, tvr)):
            view = make_tensor(owner.data + n_past * owner.nb[2], [self.d, self.hkv, n_tok],
                               list(owner.nb[:3]), op=mh.MI_OP_CPY, src=[rows])
            view.view_src = ctypes.pointer(owner)
            view.view_offs = n_past * owner.nb[2]
            cpys.append(view)
        ts = make_tensor(self.scores.ctypes.data, *nb_of(self.scores.shape, 4),
                         op=mh.MI_OP_ATTN_QK, src=[tq, self.tk], params=[n_past, self.h // self.hkv])
        tp = make_tensor(self.probs.ctypes.data, *nb_of(self.probs.shape, 4),
                         op=mh.MI_OP_SOFTMAX, src=[ts], params=[n_past, scale])
        to = make_tensor(self.out.ctypes.data, *nb_of(self.out.shape, 4),
                         op=mh.MI_OP_ATTN_KQV, src=[tp, self.tv], params=[self.h // self.hkv])
        nodes = cpys + [ts, tp, to]
        keep += [tq, tkr, tvr] + nodes
        arr = (ctypes.POINTER(mh.MiTensor) * len(nodes))(*[ctypes.pointer(n) for n in nodes])
        g = mh.MiCgraph()
        g.nodes = arr
        g.n_nodes = len(nodes)
        g.exec_nodes = arr
        g.n_exec_nodes = len(nodes)
        g.capacity = len(nodes)
        self.graph, self.nodes, self._keep = g, nodes, (keep, arr)
        return g

    def run(self, nth):
        self.hip.check(self.hip.mi_hip_graph_prepare(ctypes.byref(self.graph)))
        for node in self.nodes:
            # every worker calls the hook; only ith == 0 does the work
            for ith in reversed(range(nth)):
                rc = self.hip.mi_hip_compute_forward(ctypes.byref(node), ith, nth)
                if rc < 0:
                    raise mh.MiHipError(rc, self.hip.last_error())
                assert rc == 1, f"node op {node.op} not handled"
        return self.out


def test_executor_hook_prefill_then_decode_zero_alloc(hip, oracle):
    d, h, hkv, n_ctx = 64, 14, 2, 256
    q, k, v = cpu_attention.make_inputs(31337, d, h, hkv, n_ctx, n_ctx)
    kv = hip.kv_create(2, n_ctx, hkv, d, h)
    try:
        hg = HostGraph(hip, kv, 1, d, h, hkv, n_ctx)
        P = 40
        hg.build(q[:P], k[:P], v[:P], 0, 0.125)
        out = hg.run(nth=4)
        want = oracle.attention(q[:P], k, v, 0, 0.125, 8)[2]
        assert np.all(np.abs(out - want) <= 1e-4 + 1e-4 * np.abs(want))
        # The fused chain never materialises scores/probs on the host.
        assert np.isnan(hg.scores).all() and np.isnan(hg.probs).all()
        before = hip.alloc_stats()
        for step in range(64):
            pos = P + step
            hg.build(q[pos:pos + 1], k[pos:pos + 1], v[pos:pos + 1], pos, 0.125)
            out = hg.run(nth=2)
            if step % 21 == 0 or step == 63:
                want = oracle.attention(q[pos:pos + 1], k, v, pos, 0.125, 8)[2]
                assert np.all(np.abs(out - want) <= 1e-4 + 1e-4 * np.abs(want)), step
        after = hip.alloc_stats()
        assert after.n_malloc == before.n_malloc and after.n_free == before.n_free
        assert after.bytes_live == before.bytes_live
    finally:
        hip.check(hip.mi_hip_kv_destroy(kv))


def test_executor_hook_refuses_unplanned_device_kv(hip):
    kv = hip.kv_create(1, 64, 2, 64, 14)
    try:
        hg = HostGraph(hip, kv, 0, 64, 14, 2, 64)
        q, k, v = cpu_attention.make_inputs(1, 64, 14, 2, 64, 1)
        hg.build(q, k[:1], v[:1], 0, 0.125)
        qk = hg.nodes[2]
        # Without mi_hip_graph_prepare the hook must not let the CPU kernel read
        # the stale host copy of a device-resident cache.
        hip.check(hip.mi_hip_graph_prepare(ctypes.byref(mh.MiCgraph())))
        assert hip.mi_hip_compute_forward(ctypes.byref(qk), 0, 1) == -1
        assert "prepare" in hip.last_error()
    finally:
        hip.check(hip.mi_hip_kv_destroy(kv))


def _random_node_cases(n, seed):
    # (case, n_head_kv, n_rep, head_dim, n_past, n_tokens, f16, scale): the node
    # kernels take any head_dim, so the shapes include ones the fused kernels
    # do not (4..128)
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(rng.integers(1, 5))
        n_rep = int(rng.integers(1, 9))
        d = int(rng.choice([4, 8, 16, 32, 64, 80, 96, 128]))
        n_kv = max(1, int(np.exp(rng.uniform(0.0, np.log(700.0)))))
        n_tok = 1 if rng.uniform() < 0.5 or n_kv == 1 else int(rng.integers(2, min(n_kv, 20) + 1))
        f16 = bool(rng.integers(0, 2))
        scale = float(np.float32(1.0 / np.sqrt(d)))
        out.append((i, hkv, n_rep, d, n_kv - n_tok, n_tok, f16, scale))
    return out


@pytest.mark.parametrize("case", _random_node_cases(24, 20261205), ids=lambda c: f"n{c[0]}")
def test_node_ops_random_shapes_bit_for_bit(hip, stream, case):
    import torch
    i, hkv, n_rep, d, n_past, n_tok, f16, scale = case
    print(f"node case {i}: n_head_kv {hkv} n_rep {n_rep} D {d} n_past {n_past} n_tokens {n_tok} f16 {f16}",
          flush=True)
    n_head, n_kv = hkv * n_rep, n_past + n_tok
    q, k, v = cpu_attention.make_inputs(4000 + i, d, n_head, hkv, n_kv, n_tok)
    dq = dev(q)
    dk = dev(k.astype(np.float16)) if f16 else dev(k)
    dv = dev(v.astype(np.float16)) if f16 else dev(v)
    kt = mh.MI_TYPE_F16 if f16 else mh.MI_TYPE_F32
    elt = 2 if f16 else 4
    tq, tk, tv = dtensor(dq), dtensor(dk, elt, kt), dtensor(dv, elt, kt)
    scores = torch.full((n_head, n_tok, n_kv), float("nan"), device="cuda")
    probs = torch.full_like(scores, float("nan"))
    out = torch.full((n_tok, n_head, d), float("nan"), device="cuda")
    ts = dtensor(scores, op=mh.MI_OP_ATTN_QK, src=[tq, tk], params=[n_past, n_rep])
    tp = dtensor(probs, op=mh.MI_OP_SOFTMAX, src=[ts], params=[n_past, scale])
    to = dtensor(out, op=mh.MI_OP_ATTN_KQV, src=[tp, tv], params=[n_rep])
    hip.check(hip.mi_hip_op_attn_qk(ctypes.byref(ts), stream))
    hip.check(hip.mi_hip_op_softmax(ctypes.byref(tp), stream))
    hip.check(hip.mi_hip_op_attn_kqv(ctypes.byref(to), stream))
    torch.cuda.synchronize()
    if f16:
        k = cpu_attention.fp16_widen(k.astype(np.float16))
        v = cpu_attention.fp16_widen(v.astype(np.float16))
    want_s, want_p, want_o = cpu_attention.oracle().attention(q, k, v, n_past, scale, 4)
    assert np.array_equal(bits(scores.cpu().numpy()), bits(want_s)), f"node case {i}: scores differ"
    assert np.array_equal(bits(probs.cpu().numpy()), bits(want_p)), f"node case {i}: probs differ"
    assert np.array_equal(bits(out.cpu().numpy()), bits(want_o)), f"node case {i}: output differs"
