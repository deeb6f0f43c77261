"""Writes the golden vectors for the attention path.

Run in a container where the reference tree exists and oracle/_ref is built
(`make -C oracle all`):  python tests/golden/make_golden.py

For each case the inputs are the seeded N(0,1) draws of
oracle/cpu_attention.make_inputs (not stored: their sha256 is), and the
outputs are what the REFERENCE's own ops produce on them -- the nodes built by
src/graph.cpp:156-163, 241-253, 263-273 and executed by src/graph.cpp:75-83
(oracle/_ref/libmi_ref.so). Outputs are stored as .npz (no pickles) plus a
manifest, golden.json. F16-cache cases widen the rounded cache with the
reference's own converter (src/quant.cpp:26-63) before running the F32 ops,
which is the engine's semantics for an F16 cache.
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.cpu_attention import make_inputs, reference, sha256  # noqa: E402

OUT_DIR = os.path.dirname(os.path.abspath(__file__))

# name: (seed, head_dim, n_head, n_head_kv, n_ctx, n_past, n_tokens, kv_type)
CASES = {
    # Qwen2.5-0.5B decode at n_kv = 512 (the CPU-runnable parity config).
    "c1_decode": (1235, 64, 14, 2, 512, 511, 1, "f32"),
    # Cache longer than the visible prefix: reads honour nb[2] and stop at n_kv.
    "decode_long_ctx": (2001, 64, 14, 2, 640, 200, 1, "f32"),
    # A single visible key: the probability is exactly 1.
    "decode_one_key": (2002, 64, 14, 2, 8, 0, 1, "f32"),
    # Prefill at the 0.5B head shape (lower-triangular mask), short.
    "prefill_qwen05_short": (1237, 64, 14, 2, 40, 0, 40, "f32"),
    # Chunked prefill: n_past > 0 and n_tokens > 1 (mask boundary n_past + j).
    "prefill_chunked": (2003, 64, 4, 2, 64, 13, 19, "f32"),
    # Shapes of tests/fixtures/tiny_qwen2.gguf (n_rep 2, head_dim 4).
    "tiny_prefill": (2004, 4, 2, 1, 16, 0, 5, "f32"),
    "tiny_decode": (2005, 4, 2, 1, 16, 5, 1, "f32"),
    # Qwen2.5-7B head shape with an F16 cache, short.
    "c4_f16_decode": (1238, 128, 28, 4, 300, 299, 1, "f16"),
    # Plain multi-head (n_rep 1) prefill.
    "mha_prefill": (2006, 64, 4, 4, 48, 0, 33, "f32"),
    # Wider group (n_rep 8) decode.
    "nrep8_decode": (2007, 64, 16, 2, 200, 130, 1, "f32"),
    # head_dim 128 chunked prefill, n_rep 4.
    "d128_prefill": (2008, 128, 8, 2, 80, 7, 45, "f32"),
    # F16 cache, prefill, n_rep 7, head_dim 64.
    "f16_prefill": (2009, 64, 14, 2, 70, 3, 37, "f16"),
}

STORE_SCORES_MAX = 65536  # elements; larger cases keep only the output


# name: (head_dim, n_head, n_tokens, n_past, n_dims, freq_base, fixed input or None)
ROPE_CASES = {
    "rope_kat_identity": (4, 1, 1, 0, 4, 10000.0, [1, 2, 3, 4]),  # test_ops_cpu.cpp:181-196
    "rope_kat_rotation": (2, 1, 1, 5, 2, 10000.0, [1, 0]),        # test_ops_cpu.cpp:198-213
    "rope_q_decode": (64, 14, 1, 511, 64, 1000000.0, None),        # Qwen2.5-0.5B decode Q
    "rope_q_prefill": (64, 14, 40, 0, 64, 1000000.0, None),
    "rope_k_chunk": (64, 2, 19, 13, 64, 1000000.0, None),          # a chunk after 13 tokens
    "rope_7b_q_far": (128, 28, 2, 30000, 128, 1000000.0, None),    # large angles
    "rope_partial": (64, 4, 3, 5, 32, 10000.0, None),              # n_dims < head_dim
}


# name: (k, n rows, m columns) of MI_OP_MUL_MAT with Q8_0 weights
Q8_CASES = {
    "q8_kat": (64, 5, 4),
    "q8_oproj_rows": (896, 64, 3),    # Qwen2.5-0.5B attn_output k, 64 of its 896 rows
    "q8_ffn_down_rows": (4864, 24, 2),  # ffn_down k = 4864
}


def x_ptr(a):
    return a.ctypes.data


def f16_lut(ref):
    import ctypes
    fn = ref.lib.ref_fp16_to_fp32_row
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
    codes = np.arange(65536, dtype=np.uint16)
    lut = np.empty(65536, np.float32)
    fn(codes.ctypes.data, lut.ctypes.data, 65536)
    return lut


def main():
    ref = reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libmi_ref.so is missing: run make -C oracle all")
    lut = None
    manifest = {"generator": "tests/golden/make_golden.py", "cases": {}}
    for name, (seed, d, h, hkv, n_ctx, n_past, t, kv_type) in CASES.items():
        q, k, v = make_inputs(seed, d, h, hkv, n_ctx, t)
        entry = {"seed": seed, "head_dim": d, "n_head": h, "n_head_kv": hkv, "n_ctx": n_ctx,
                 "n_past": n_past, "n_tokens": t, "kv_type": kv_type,
                 "scale": float(np.float32(1.0) / np.sqrt(np.float32(d))),
                 "sha256_q": sha256(q), "sha256_k": sha256(k), "sha256_v": sha256(v)}
        kk, vv = k, v
        if kv_type == "f16":
            if lut is None:
                lut = f16_lut(ref)
            kk = lut[k.astype(np.float16).view(np.uint16)]
            vv = lut[v.astype(np.float16).view(np.uint16)]
        scale = np.float32(entry["scale"])
        scores, probs, out = ref.attention(q, kk, vv, n_past, float(scale), n_threads=3)
        arrays = {"out": out}
        if scores.size <= STORE_SCORES_MAX:
            arrays["scores"] = scores
            arrays["probs"] = probs
        entry["sha256"] = {key: sha256(a) for key, a in arrays.items()}
        np.savez(os.path.join(OUT_DIR, name + ".npz"), **arrays)
        manifest["cases"][name] = entry
        print(f"{name}: out {out.shape} max|out| {np.abs(out).max():.4f}")

    # Known-answer softmax of tests/test_ops_cpu.cpp:215-241 (masked 99s).
    src = np.array([[[5, 99, 99, 99], [1, 3, 99, 99]]], dtype=np.float32)  # [h=1][j=2][i=4]
    dst = np.empty_like(src)
    fn = ref.lib.ref_softmax
    import ctypes
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 4 + [ctypes.c_float]
    fn(src.ctypes.data, dst.ctypes.data, 4, 2, 1, 0, ctypes.c_float(1.0))
    np.savez(os.path.join(OUT_DIR, "softmax_kat.npz"), src=src, probs=dst)
    manifest["softmax_kat"] = {"n_past": 0, "scale": 1.0, "sha256_probs": sha256(dst)}

    # MI_OP_ROPE (src/ops_cpu.cpp:270-302): the known-answer cases of
    # tests/test_ops_cpu.cpp:181-213 and the engine's Q/K shapes, inputs
    # [n_tokens][n_head][head_dim] from a seeded generator, stored with them.
    import ctypes
    fn = ref.lib.ref_rope
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 5 + [ctypes.c_float]
    rng = np.random.default_rng(4242)
    manifest["rope"] = {}
    for name, (d, h, t, n_past, n_dims, base, src) in ROPE_CASES.items():
        x = (np.asarray(src, np.float32).reshape(t, h, d) if src is not None
             else rng.standard_normal((t, h, d)).astype(np.float32))
        y = np.empty_like(x)
        fn(x.ctypes.data, y.ctypes.data, d, h, t, n_past, n_dims, ctypes.c_float(base))
        np.savez(os.path.join(OUT_DIR, name + ".npz"), src=x, dst=y)
        manifest["rope"][name] = {"head_dim": d, "n_head": h, "n_tokens": t, "n_past": n_past,
                                  "n_dims": n_dims, "freq_base": base,
                                  "sha256_src": sha256(x), "sha256_dst": sha256(y)}
        print(f"{name}: {x.shape}")

    # Q8_0 (src/quant.cpp): weight rows from seeded N(0, 0.02) floats, the
    # activation quantized by the reference, and mul_mat's dot products as the
    # reference dispatches them. Row/column counts kept small (fixtures).
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    ref.lib.ref_quantize_rows_q8_0.argtypes = [vp, vp, i64, i64]
    ref.lib.ref_quantize_rows_q8_0_act.argtypes = [vp, vp, i64, i64]
    ref.lib.ref_mul_mat_q8_0.argtypes = [vp, vp, vp, i64, i64, i64]
    manifest["q8_0"] = {}
    rng = np.random.default_rng(8080)
    for name, (k, n, m) in Q8_CASES.items():
        wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        x = rng.standard_normal((m, k)).astype(np.float32)
        if name == "q8_kat":
            x[0, :32] = 0.0                                   # all-zero block: d = 0, q = 0
            x[1, :32] = np.arange(32, dtype=np.float32) - 15.5  # ties at .5 (amax 15.5)
            x[1, 31] = 127.0                                   # amax 127 -> d = 1, ties stay ties
            x[2, 32:64] = -x[2, 32:64]
        w = np.empty(n * (k // 32) * 34, np.uint8)
        ref.lib.ref_quantize_rows_q8_0(x_ptr(wf), w.ctypes.data, k, n)
        act = np.empty(m * (k // 32) * 36, np.uint8)
        ref.lib.ref_quantize_rows_q8_0_act(x_ptr(x), act.ctypes.data, k, m)
        dst = np.empty((m, n), np.float32)
        ref.lib.ref_mul_mat_q8_0(w.ctypes.data, act.ctypes.data, dst.ctypes.data, k, n, m)
        np.savez(os.path.join(OUT_DIR, name + ".npz"), w=w, x=x, act=act, dst=dst)
        manifest["q8_0"][name] = {"k": k, "n": n, "m": m, "sha256_w": sha256(w),
                                  "sha256_x": sha256(x), "sha256_act": sha256(act),
                                  "sha256_dst": sha256(dst)}
        print(f"{name}: k={k} n={n} m={m}")

    # The reference's F16 widening over every code, as float32 bit patterns.
    if lut is None:
        lut = f16_lut(ref)
    manifest["fp16_lut_sha256"] = sha256(lut.view(np.uint32))

    with open(os.path.join(OUT_DIR, "golden.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote", len(CASES), "cases")


if __name__ == "__main__":
    main()
