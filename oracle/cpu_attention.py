"""ctypes front end of the CPU checker libraries.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, never by the product library.

Two interchangeable back ends with the same calls:
  oracle()    -> oracle/liboracle_attn.so, this repository's restatement of
                 src/ops_cpu.cpp:304-410 (always built by oracle/Makefile);
  reference() -> oracle/_ref/libmi_ref.so, the reference's own sources compiled
                 in place (only where the reference tree was present at build
                 time); None when absent.

Array conventions (numpy C order, i.e. reversed engine ne[]):
  q   (n_tokens, n_head, head_dim)      == engine [head_dim, n_head, n_tokens]
  k,v (n_ctx, n_head_kv, head_dim)      == engine [head_dim, n_head_kv, n_ctx]
  scores, probs (n_head, n_tokens, n_kv) == engine [n_kv, n_tokens, n_head]
  out (n_tokens, n_head, head_dim)      == engine [head_dim, n_head, n_tokens]
"""
import ctypes
import hashlib
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle_attn.so")
REF_SO = os.path.join(HERE, "_ref", "libmi_ref.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_pp = ctypes.POINTER(ctypes.c_void_p)


def _ptr(a):
    return a.ctypes.data_as(_f32p)


def make_inputs(seed, head_dim, n_head, n_head_kv, n_ctx, n_tokens):
    """Seeded i.i.d. N(0,1) float32 Q, K, V (PCG64, drawn in that order)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n_tokens, n_head, head_dim), dtype=np.float32)
    k = rng.standard_normal((n_ctx, n_head_kv, head_dim), dtype=np.float32)
    v = rng.standard_normal((n_ctx, n_head_kv, head_dim), dtype=np.float32)
    return q, k, v


def sha256(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


class CpuAttention:
    def __init__(self, path, prefix):
        self.path = path
        self.kind = "reference" if prefix == "ref" else "port"
        lib = ctypes.CDLL(path)
        self.lib = lib
        args = [_f32p] * 6 + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int]
        self._attention = getattr(lib, prefix + "_attention")
        self._attention.argtypes = args
        self._attention.restype = ctypes.c_int
        self._time = getattr(lib, prefix + "_time_attention")
        self._time.argtypes = [_pp, _pp, _pp, _f32p, _f32p, _pp] + [ctypes.c_int] * 7 + [
            ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        self._time.restype = ctypes.c_double
        self._f16 = getattr(lib, prefix + "_fp16_to_fp32")
        self._f16.argtypes = [ctypes.c_uint16]
        self._f16.restype = ctypes.c_float

    def attention(self, q, k, v, n_past, scale, n_threads=1):
        """Returns (scores, probs, out) of the three-node pass."""
        n_tokens, n_head, head_dim = q.shape
        n_ctx, n_head_kv, _ = k.shape
        n_kv = n_past + n_tokens
        q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
        scores = np.empty((n_head, n_tokens, n_kv), np.float32)
        probs = np.empty_like(scores)
        out = np.empty((n_tokens, n_head, head_dim), np.float32)
        rc = self._attention(_ptr(q), _ptr(k), _ptr(v), _ptr(scores), _ptr(probs), _ptr(out),
                             head_dim, n_head, n_head_kv, n_ctx, n_past, n_tokens,
                             ctypes.c_float(scale), n_threads)
        if rc != 0:
            raise ValueError("inconsistent attention sizes")
        return scores, probs, out

    def fp16_to_fp32(self, h):
        return self._f16(h)

    def time_attention(self, qs, ks, vs, n_past, scale, n_threads, warmup=1, reps=5):
        """Median seconds for len(qs) layers' three-node passes (one graph)."""
        n_layers = len(qs)
        n_tokens, n_head, head_dim = qs[0].shape
        n_ctx, n_head_kv, _ = ks[0].shape
        n_kv = n_past + n_tokens
        scores = np.empty((n_head, n_tokens, n_kv), np.float32)
        probs = np.empty_like(scores)
        outs = [np.empty((n_tokens, n_head, head_dim), np.float32) for _ in range(n_layers)]
        arr = lambda xs: (ctypes.c_void_p * n_layers)(*[x.ctypes.data for x in xs])
        t = self._time(arr(qs), arr(ks), arr(vs), _ptr(scores), _ptr(probs), arr(outs), n_layers,
                       head_dim, n_head, n_head_kv, n_ctx, n_past, n_tokens,
                       ctypes.c_float(scale), n_threads, warmup, reps)
        if t < 0:
            raise ValueError("inconsistent attention sizes")
        return t, outs


class Oracle(CpuAttention):
    """The restatement, plus its node-level entry points."""

    def __init__(self):
        super().__init__(ORACLE_SO, "oracle")
        self.lib.oracle_split_range.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                                ctypes.POINTER(ctypes.c_int64),
                                                ctypes.POINTER(ctypes.c_int64)]

    def rope(self, x, n_past, n_dims, freq_base):
        """MI_OP_ROPE of x shaped (n_tokens, n_head, head_dim), one thread."""
        x = np.ascontiguousarray(x, np.float32)
        t, h, d = x.shape
        y = np.empty_like(x)
        fn = self.lib.oracle_rope
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 5 + [ctypes.c_float]
        fn(x.ctypes.data, y.ctypes.data, d, h, t, n_past, n_dims, ctypes.c_float(freq_base))
        return y

    def quantize_q8_0_act(self, x):
        """Activation rows x (m, k) -> raw Q8_0_ACT blocks (m * k/32 * 36 bytes)."""
        x = np.ascontiguousarray(x, np.float32)
        m, k = x.shape
        out = np.empty(m * (k // 32) * 36, np.uint8)
        fn = self.lib.oracle_quantize_q8_0_act
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
        fn(x.ctypes.data, out.ctypes.data, k, m)
        return out

    def mul_mat_q8_0(self, w, act, k, n, m):
        """Raw Q8_0 weight rows (n x k/32 blocks) . raw activation blocks -> (m, n)."""
        dst = np.empty((m, n), np.float32)
        fn = self.lib.oracle_mul_mat_q8_0_contig
        fn.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3
        fn(np.ascontiguousarray(w).ctypes.data, np.ascontiguousarray(act).ctypes.data,
           dst.ctypes.data, k, n, m)
        return dst

    def split_range(self, n, ith, nth):
        lo, hi = ctypes.c_int64(), ctypes.c_int64()
        self.lib.oracle_split_range(n, ith, nth, ctypes.byref(lo), ctypes.byref(hi))
        return lo.value, hi.value


_cache = {}


def oracle():
    if "oracle" not in _cache:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle/liboracle_attn.so is not built (run make -C oracle)")
        _cache["oracle"] = Oracle()
    return _cache["oracle"]


def reference():
    if "ref" not in _cache:
        _cache["ref"] = CpuAttention(REF_SO, "ref") if os.path.exists(REF_SO) else None
    return _cache["ref"]


def fp16_widen(k16):
    """Exact float16 -> float32 via the restatement's converter (LUT over all
    65536 codes), the F16-cache oracle of the engine's F32 ops."""
    lut = _fp16_lut()
    return lut[np.ascontiguousarray(k16).view(np.uint16)]


def _fp16_lut():
    if "lut" not in _cache:
        o = oracle()
        lut = np.empty(65536, np.float32)
        codes = np.arange(65536, dtype=np.uint16)
        fn = o.lib.oracle_fp16_to_fp32_row
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        fn(codes.ctypes.data, lut.ctypes.data, 65536)
        _cache["lut"] = lut
    return _cache["lut"]


def q8_weight_blocks(w_raw, n, k):
    """Raw Q8_0 weight rows -> (fp16 scales (n, k/32), int8 values (n, k/32, 32))."""
    b = np.ascontiguousarray(w_raw).view(np.uint8).reshape(n, k // 32, 34)
    d = b[:, :, :2].copy().view(np.float16)[:, :, 0]
    return d, b[:, :, 2:].copy().view(np.int8)


def q8_act_blocks(a_raw, m, k):
    """Raw Q8_0_ACT rows -> (float scales (m, k/32), int8 values (m, k/32, 32))."""
    b = np.ascontiguousarray(a_raw).view(np.uint8).reshape(m, k // 32, 36)
    d = b[:, :, :4].copy().view(np.float32)[:, :, 0]
    return d, b[:, :, 4:].copy().view(np.int8)
