"""ctypes binding of libmi_hip_attn.so (the C ABI of include/mi_hip_attn.h).

This is a thin test/benchmark front end: the product is the C ABI itself.
Device memory comes from torch (torch.cuda tensors on ROCm); only raw device
addresses cross into the library. Loading fails loudly when the library has
not been built -- there is no fallback path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmi_hip_attn.so")

MI_TYPE_F32 = 0
MI_TYPE_F16 = 1
MI_TYPE_Q8_0 = 2
MI_TYPE_Q8_0_ACT = 4

MI_OP_NONE = 0
MI_OP_MUL_MAT = 5
MI_OP_ROPE = 6
MI_OP_SOFTMAX = 7
MI_OP_CPY = 10
MI_OP_QUANTIZE_Q8_0 = 11
MI_OP_VIEW = 13
MI_OP_ATTN_QK = 16
MI_OP_ATTN_KQV = 17

MI_TENSOR_FLAG_KV = 1 << 3

MI_HIP_PREFILL_F32 = 0
MI_HIP_PREFILL_SPLIT_BF16 = 1
MI_HIP_PREFILL_AUTO = 2
MI_HIP_DECODE_VALU = 0
MI_HIP_DECODE_MATRIX = 1
MI_HIP_DECODE_AUTO = 2
MI_HIP_DECODE_STREAM = 3

MI_HIP_QWEN2_ATTN_FUSED = 0
MI_HIP_QWEN2_ATTN_REFERENCE_ORDER = 1

STATUS = {0: "OK", 1: "E_INVALID", 2: "E_NODEVICE", 3: "E_RUNTIME", 4: "E_NOMEM",
          5: "E_UNSUPPORTED", 6: "E_STATE", 7: "E_LOST"}


class MiHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


class MiTensor(ctypes.Structure):
    """ABI mirror of struct mi_tensor (src/tensor.h:122-160)."""


MiTensor._fields_ = [
    ("type", ctypes.c_int),
    ("ne", ctypes.c_int64 * 4),
    ("nb", ctypes.c_size_t * 4),
    ("op", ctypes.c_int),
    ("op_params", ctypes.c_int32 * 8),
    ("src", ctypes.POINTER(MiTensor) * 2),
    ("data", ctypes.c_void_p),
    ("view_src", ctypes.POINTER(MiTensor)),
    ("view_offs", ctypes.c_size_t),
    ("n_children", ctypes.c_int32),
    ("flags", ctypes.c_uint32),
    ("name", ctypes.c_char * 64),
    ("extra", ctypes.c_void_p),
]


class MiCgraph(ctypes.Structure):
    _fields_ = [
        ("nodes", ctypes.POINTER(ctypes.POINTER(MiTensor))),
        ("n_nodes", ctypes.c_int),
        ("leafs", ctypes.POINTER(ctypes.POINTER(MiTensor))),
        ("n_leafs", ctypes.c_int),
        ("exec_nodes", ctypes.POINTER(ctypes.POINTER(MiTensor))),
        ("n_exec_nodes", ctypes.c_int),
        ("capacity", ctypes.c_int),
    ]


class KvDesc(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int32), ("n_ctx", ctypes.c_int32),
                ("n_head_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("n_head", ctypes.c_int32), ("type", ctypes.c_int32)]


class WorkspaceDesc(ctypes.Structure):
    _fields_ = [("n_head_kv", ctypes.c_int32), ("n_head", ctypes.c_int32),
                ("head_dim", ctypes.c_int32)]


class WorkspaceStatus(ctypes.Structure):
    _fields_ = [("early_fallbacks", ctypes.c_uint32), ("lost_groups", ctypes.c_uint32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("kv", ctypes.c_void_p),
        ("layer", ctypes.c_int32),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_nb", ctypes.c_size_t * 3),
        ("v_nb", ctypes.c_size_t * 3),
        ("kv_type", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("n_head_kv", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("q_nb", ctypes.c_size_t * 3),
        ("out", ctypes.c_void_p),
        ("out_nb", ctypes.c_size_t * 3),
        ("n_head", ctypes.c_int32),
        ("n_rep", ctypes.c_int32),
        ("n_past", ctypes.c_int32),
        ("n_tokens", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("stream", ctypes.c_void_p),
        ("ws", ctypes.c_void_p),
    ]


class RopeArgs(ctypes.Structure):
    _fields_ = [
        ("kv", ctypes.c_void_p),
        ("layer", ctypes.c_int32),
        ("n_past", ctypes.c_int32),
        ("n_tokens", ctypes.c_int32),
        ("n_dims", ctypes.c_int32),
        ("freq_base", ctypes.c_float),
        ("n_head", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("q_nb", ctypes.c_size_t * 3),
        ("q_out", ctypes.c_void_p),
        ("q_out_nb", ctypes.c_size_t * 3),
        ("k", ctypes.c_void_p),
        ("k_nb", ctypes.c_size_t * 3),
        ("v", ctypes.c_void_p),
        ("v_nb", ctypes.c_size_t * 3),
        ("stream", ctypes.c_void_p),
    ]


class Qwen2Hparams(ctypes.Structure):
    """ABI mirror of mi_hip_qwen2_hparams (include/mi_hip_qwen2.h)."""
    _fields_ = [("n_vocab", ctypes.c_int32), ("n_embd", ctypes.c_int32),
                ("n_layer", ctypes.c_int32), ("n_head", ctypes.c_int32),
                ("n_head_kv", ctypes.c_int32), ("n_ff", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("n_ctx_train", ctypes.c_int32),
                ("rope_freq_base", ctypes.c_float), ("rms_eps", ctypes.c_float)]


class AllocStats(ctypes.Structure):
    _fields_ = [("n_malloc", ctypes.c_uint64), ("n_free", ctypes.c_uint64),
                ("bytes_live", ctypes.c_uint64), ("bytes_peak", ctypes.c_uint64)]


# Every symbol include/mi_hip_attn.h and include/mi_hip_qwen2.h declare, with
# its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
SIGNATURES = {
    "mi_hip_init": ([_I], _I),
    "mi_hip_shutdown": ([], _I),
    "mi_hip_last_error": ([], ctypes.c_char_p),
    "mi_hip_abi_layout": ([ctypes.POINTER(ctypes.c_size_t), _I], _I),
    "mi_hip_get_alloc_stats": ([ctypes.POINTER(AllocStats)], _I),
    "mi_hip_set_alloc_limit": ([ctypes.c_uint64], _I),
    "mi_hip_kv_create": ([ctypes.POINTER(KvDesc), ctypes.POINTER(ctypes.c_void_p)], _I),
    "mi_hip_kv_destroy": ([_P], _I),
    "mi_hip_kv_workspace": ([_P, ctypes.POINTER(ctypes.c_void_p)], _I),
    "mi_hip_workspace_create": ([ctypes.POINTER(WorkspaceDesc), ctypes.POINTER(ctypes.c_void_p)], _I),
    "mi_hip_workspace_destroy": ([_P], _I),
    "mi_hip_workspace_check": ([_P, _P, ctypes.POINTER(WorkspaceStatus)], _I),
    "mi_hip_workspace_set_poll_limit": ([_P, ctypes.c_int32], _I),
    "mi_hip_set_deterministic": ([ctypes.c_int32], _I),
    "mi_hip_set_prefill_mode": ([ctypes.c_int32], _I),
    "mi_hip_set_decode_mode": ([ctypes.c_int32], _I),
    "mi_hip_set_host_nodes": ([ctypes.c_int32], _I),
    "mi_hip_decode_tuning": ([ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32], _I),
    "mi_hip_kv_view": ([_P, _I, _I, ctypes.POINTER(ctypes.c_void_p),
                        ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_size_t)], _I),
    "mi_hip_kv_write": ([_P, _I, _I, _I, _I, _P, ctypes.POINTER(ctypes.c_size_t), _I, _P], _I),
    "mi_hip_kv_bind": ([_P, _I, _I, ctypes.POINTER(MiTensor)], _I),
    "mi_hip_attn_fwd": ([ctypes.POINTER(AttnArgs)], _I),
    "mi_hip_attn_fwd_reference_order": ([ctypes.POINTER(AttnArgs)], _I),
    "mi_hip_attn_decode_batch": ([ctypes.POINTER(AttnArgs), _I, _P], _I),
    "mi_hip_attn_decode_batch_noalloc": ([ctypes.POINTER(AttnArgs), _I, _P], _I),
    "mi_hip_op_attn_qk": ([ctypes.POINTER(MiTensor), _P], _I),
    "mi_hip_op_softmax": ([ctypes.POINTER(MiTensor), _P], _I),
    "mi_hip_op_attn_kqv": ([ctypes.POINTER(MiTensor), _P], _I),
    "mi_hip_op_attn_fused": ([ctypes.POINTER(MiTensor), _P], _I),
    "mi_hip_op_rope": ([ctypes.POINTER(MiTensor), _P], _I),
    "mi_hip_op_quantize_q8_0": ([ctypes.POINTER(MiTensor), _P], _I),
    "mi_hip_op_mul_mat": ([ctypes.POINTER(MiTensor), _P], _I),
    "mi_hip_rope_append": ([ctypes.POINTER(RopeArgs)], _I),
    "mi_hip_memread": ([_P, ctypes.c_size_t, _P, ctypes.c_int32, _P], _I),
    "mi_hip_graph_prepare": ([ctypes.POINTER(MiCgraph)], _I),
    "mi_hip_compute_forward": ([ctypes.POINTER(MiTensor), _I, _I], _I),
    "mi_hip_qwen2_load": ([ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32,
                           ctypes.POINTER(ctypes.c_void_p)], _I),
    "mi_hip_qwen2_free": ([_P], _I),
    "mi_hip_qwen2_get_hparams": ([_P, ctypes.POINTER(Qwen2Hparams)], _I),
    "mi_hip_qwen2_forward": ([_P, ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, ctypes.c_int32,
                              ctypes.c_int32, ctypes.POINTER(ctypes.c_float),
                              ctypes.POINTER(ctypes.c_int32)], _I),
    "mi_hip_qwen2_generate": ([_P, ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, ctypes.c_int32,
                               ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)], _I),
    "mi_hip_qwen2_set_attention": ([_P, ctypes.c_int32], _I),
    "mi_hip_qwen2_set_timing": ([_P, ctypes.c_int32], _I),
    "mi_hip_qwen2_get_timing": ([_P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(ctypes.c_int64)], _I),
}


class Lib:
    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built: run `make -C mini-infer-llama.cpp_amd` "
                               "(or __graft_entry__.build())")
        self.path = path
        self.so = ctypes.CDLL(path)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(self.so, name)
            fn.argtypes = argtypes
            fn.restype = restype

    def last_error(self):
        return self.so.mi_hip_last_error().decode()

    def check(self, rc):
        if rc != 0:
            raise MiHipError(rc, self.last_error())
        return rc

    def __getattr__(self, name):
        return getattr(self.so, name)

    # -- convenience wrappers -------------------------------------------------
    def init(self, device=0):
        self.check(self.so.mi_hip_init(device))

    def alloc_stats(self):
        s = AllocStats()
        self.check(self.so.mi_hip_get_alloc_stats(ctypes.byref(s)))
        return s

    def abi_layout(self):
        arr = (ctypes.c_size_t * 15)()
        self.check(self.so.mi_hip_abi_layout(arr, 15))
        return list(arr)

    def kv_create(self, n_layer, n_ctx, n_head_kv, head_dim, n_head, kv_type=MI_TYPE_F32):
        d = KvDesc(n_layer, n_ctx, n_head_kv, head_dim, n_head, kv_type)
        h = ctypes.c_void_p()
        self.check(self.so.mi_hip_kv_create(ctypes.byref(d), ctypes.byref(h)))
        return h.value

    def workspace_create(self, n_head_kv, n_head, head_dim):
        d = WorkspaceDesc(n_head_kv, n_head, head_dim)
        h = ctypes.c_void_p()
        self.check(self.so.mi_hip_workspace_create(ctypes.byref(d), ctypes.byref(h)))
        return h.value

    def kv_workspace(self, kv):
        h = ctypes.c_void_p()
        self.check(self.so.mi_hip_kv_workspace(kv, ctypes.byref(h)))
        return h.value

    def workspace_check(self, ws, stream):
        """(status code, early_fallbacks, lost_groups) since the last check."""
        st = WorkspaceStatus()
        rc = self.so.mi_hip_workspace_check(ws, stream, ctypes.byref(st))
        return rc, st.early_fallbacks, st.lost_groups

    def kv_view(self, kv, layer, which):
        data = ctypes.c_void_p()
        ne = (ctypes.c_int64 * 4)()
        nb = (ctypes.c_size_t * 4)()
        self.check(self.so.mi_hip_kv_view(kv, layer, which, ctypes.byref(data), ne, nb))
        return data.value, list(ne), list(nb)


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = Lib()
    return _lib


def nb3_of(t):
    """Byte strides (ne[0] innermost) of a torch tensor shaped (ne2, ne1, ne0)."""
    es = t.element_size()
    s = t.stride()
    return (s[2] * es, s[1] * es, s[0] * es)


def attn_args(q, out, n_rep, n_past, scale, stream, kv=None, layer=0, k=None, v=None, ws=None):
    """Builds AttnArgs from torch tensors q/out shaped (n_tokens, n_head, head_dim) and
    either a cache handle + layer or explicit k/v shaped (n_ctx, n_head_kv, head_dim);
    ws: an optional decode workspace handle (else the cache's, else the library default)."""
    a = AttnArgs()
    a.ws = ws
    if kv is not None:
        a.kv = kv
        a.layer = layer
    else:
        import torch
        a.k, a.v = k.data_ptr(), v.data_ptr()
        a.k_nb[:] = nb3_of(k)
        a.v_nb[:] = nb3_of(v)
        a.kv_type = MI_TYPE_F16 if k.dtype == torch.float16 else MI_TYPE_F32
        a.head_dim = k.shape[2]
        a.n_head_kv = k.shape[1]
    a.q = q.data_ptr()
    a.q_nb[:] = nb3_of(q)
    a.out = out.data_ptr()
    a.out_nb[:] = nb3_of(out)
    a.n_tokens, a.n_head = q.shape[0], q.shape[1]
    a.n_rep = n_rep
    a.n_past = n_past
    a.scale = scale
    a.stream = stream
    return a


def rope_args(kv, layer, n_past, n_dims, freq_base, stream, k, v, q=None, q_out=None):
    """Builds RopeArgs from torch tensors shaped (n_tokens, heads, head_dim): k/v
    with the cache's n_head_kv heads, q/q_out (optional) with n_head heads."""
    a = RopeArgs()
    a.kv, a.layer, a.n_past, a.n_dims = kv, layer, n_past, n_dims
    a.freq_base = freq_base
    a.n_tokens = k.shape[0]
    a.k, a.v = k.data_ptr(), v.data_ptr()
    a.k_nb[:] = nb3_of(k)
    a.v_nb[:] = nb3_of(v)
    if q is not None:
        q_out = q if q_out is None else q_out
        a.q, a.q_out = q.data_ptr(), q_out.data_ptr()
        a.q_nb[:] = nb3_of(q)
        a.q_out_nb[:] = nb3_of(q_out)
        a.n_head = q.shape[1]
    a.stream = stream
    return a


def make_tensor(data_ptr, ne, nb, type_=MI_TYPE_F32, op=MI_OP_NONE, src=(), params=()):
    """An mi_tensor descriptor (ne/nb in engine order, ne[0] innermost)."""
    t = MiTensor()
    t.type = type_
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    t.ne[:] = ne
    t.nb[:] = nb
    t.op = op
    t.data = data_ptr
    for i, s in enumerate(src):
        t.src[i] = ctypes.pointer(s)
    for i, p in enumerate(params):
        if isinstance(p, float):
            t.op_params[i] = ctypes.c_int32.from_buffer(ctypes.c_float(p)).value
        else:
            t.op_params[i] = p
    return t
