"""Random-initialised Qwen2-architecture GGUF v3 files with Q8_0 weights.

The end-to-end workload (greedy generation on a Qwen2.5-0.5B-shaped model)
needs a model file and there are no checkpoints to download, so this module
writes one from a seed. The file is what the engine's loader reads
(src/gguf.cpp:259-436, hparams src/model_qwen2.cpp:426-463, tensors :487-533,
vocabulary src/gguf.cpp:725-757):

  * header: magic "GGUF", version 3, tensor and key counts (u64);
  * keys: general.architecture, general.alignment (32), the qwen2.* hparams,
    tokenizer.ggml.tokens (one placeholder string per id);
  * tensors: token_embd.weight, output_norm.weight and per layer blk.N.*
    (by default no output.weight: the lm_head is tied to token_embd,
    :497-505), each tensor's data at a 32-byte aligned offset of the data
    section.

Values. Weight matrices and biases are N(0, 0.02), RMSNorm weights are 1.0.
The normal draws use no libm: element e of tensor t takes
h = splitmix64(seed * 2^32 + t * 2^40 + e) (a 64-bit counter hash), sums its
four 16-bit fields (Irwin-Hall, n = 4) and standardises the sum, so the file
is a pure function of the seed, identical on every machine. Matrices are then
quantised to Q8_0 (34-byte blocks: fp16 scale d = amax/127, 32 int8
round-half-to-even(x/d), src/quant.cpp:129-153, fp16 by round to nearest
even); 1-D tensors stay F32; token_embd may instead be F16 or F32 (then with
a separate Q8_0 output.weight).
"""
import hashlib
import os
import struct

import numpy as np

GGUF_ALIGN = 32
T_F32, T_F16, T_Q8_0 = 0, 1, 8  # GGUF tensor type ids (src/gguf.cpp:378-393)
KV_U32, KV_F32, KV_STRING, KV_ARRAY = 4, 6, 8, 9

QWEN2_05B = dict(n_vocab=151936, n_embd=896, n_layer=24, n_head=14, n_head_kv=2, n_ff=4864,
                 n_ctx_train=32768, rope_freq_base=1000000.0, rms_eps=1e-6)

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLD = np.uint64(0x9E3779B97F4A7C15)
_MIX1 = np.uint64(0xBF58476D1CE4E5B9)
_MIX2 = np.uint64(0x94D049BB133111EB)
# Irwin-Hall of four discrete uniforms on [0, 65535]: mean 131070, variance
# 4 * (65536^2 - 1) / 12.
_IH_MEAN = 131070.0
_IH_STD = float(np.sqrt(4.0 * (65536.0 ** 2 - 1.0) / 12.0))
STD = 0.02


def splitmix64(z):
    """splitmix64 finaliser of z + golden gamma, on a uint64 array (wraps mod 2^64)."""
    with np.errstate(over="ignore"):
        z = z + _GOLD
        z = (z ^ (z >> np.uint64(30))) * _MIX1
        z = (z ^ (z >> np.uint64(27))) * _MIX2
        return z ^ (z >> np.uint64(31))


def normal_chunk(seed, tensor_index, start, count):
    """float32 N(0, 0.02) draws for elements [start, start + count) of a tensor."""
    base = np.uint64((seed << 32) + (tensor_index << 40) + start)
    with np.errstate(over="ignore"):
        h = splitmix64(np.arange(count, dtype=np.uint64) + base)
    m = np.uint64(0xFFFF)
    s = ((h & m) + ((h >> np.uint64(16)) & m) + ((h >> np.uint64(32)) & m) + (h >> np.uint64(48)))
    return ((s.astype(np.float64) - _IH_MEAN) * (STD / _IH_STD)).astype(np.float32)


def quantize_q8_0(x):
    """Q8_0 blocks of a float32 array whose length is a multiple of 32 (src/quant.cpp:129-153)."""
    xb = x.reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1)
    d = amax / np.float32(127.0)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint(xb * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((xb.shape[0], 34), dtype=np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def prompt_ids(seed, n, n_vocab):
    """n token ids, uniform over [0, n_vocab) from the same counter hash (stream 2^63)."""
    h = splitmix64(np.arange(n, dtype=np.uint64) + np.uint64((1 << 63) + (seed << 32)))
    return (h % np.uint64(n_vocab)).astype(np.int64).tolist()


def tensor_plan(hp):
    """(name, ne, gguf type, init) in file order; init is 'normal' or 'ones'.
    hp may carry embd_type (T_Q8_0 default, T_F16 or T_F32) for token_embd;
    with a non-Q8_0 embedding a separate Q8_0 output.weight (the lm_head) is
    written after it (src/model_qwen2.cpp:497-505)."""
    E, F = hp["n_embd"], hp["n_ff"]
    hd = E // hp["n_head"]
    kv = hd * hp["n_head_kv"]
    et = hp.get("embd_type", T_Q8_0)
    plan = [("token_embd.weight", (E, hp["n_vocab"]), et, "normal"),
            ("output_norm.weight", (E,), T_F32, "ones")]
    if et != T_Q8_0:
        plan.append(("output.weight", (E, hp["n_vocab"]), T_Q8_0, "normal"))
    for l in range(hp["n_layer"]):
        b = f"blk.{l}."
        plan += [(b + "attn_norm.weight", (E,), T_F32, "ones"),
                 (b + "attn_q.weight", (E, E), T_Q8_0, "normal"),
                 (b + "attn_q.bias", (E,), T_F32, "normal"),
                 (b + "attn_k.weight", (E, kv), T_Q8_0, "normal"),
                 (b + "attn_k.bias", (kv,), T_F32, "normal"),
                 (b + "attn_v.weight", (E, kv), T_Q8_0, "normal"),
                 (b + "attn_v.bias", (kv,), T_F32, "normal"),
                 (b + "attn_output.weight", (E, E), T_Q8_0, "normal"),
                 (b + "ffn_norm.weight", (E,), T_F32, "ones"),
                 (b + "ffn_gate.weight", (E, F), T_Q8_0, "normal"),
                 (b + "ffn_up.weight", (E, F), T_Q8_0, "normal"),
                 (b + "ffn_down.weight", (F, E), T_Q8_0, "normal")]
    return plan


def _nbytes(ne, t):
    n = int(np.prod(ne))
    return n * 4 if t == T_F32 else (n * 2 if t == T_F16 else n // 32 * 34)


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _kv_u32(k, v):
    return _str(k) + struct.pack("<II", KV_U32, v)


def _kv_f32(k, v):
    return _str(k) + struct.pack("<If", KV_F32, v)


def _align(n):
    return (n + GGUF_ALIGN - 1) // GGUF_ALIGN * GGUF_ALIGN


def write_qwen2_q8_0(path, seed, hp=None, chunk=1 << 22):
    """Writes the model file; returns its sha256 (hex)."""
    hp = dict(QWEN2_05B if hp is None else hp)
    plan = tensor_plan(hp)
    kvs = [_str("general.architecture") + struct.pack("<I", KV_STRING) + _str("qwen2"),
           _kv_u32("general.alignment", GGUF_ALIGN),
           _kv_u32("qwen2.embedding_length", hp["n_embd"]),
           _kv_u32("qwen2.block_count", hp["n_layer"]),
           _kv_u32("qwen2.attention.head_count", hp["n_head"]),
           _kv_u32("qwen2.attention.head_count_kv", hp["n_head_kv"]),
           _kv_u32("qwen2.feed_forward_length", hp["n_ff"]),
           _kv_u32("qwen2.context_length", hp["n_ctx_train"]),
           _kv_f32("qwen2.rope.freq_base", hp["rope_freq_base"]),
           _kv_f32("qwen2.attention.layer_norm_rms_epsilon", hp["rms_eps"])]
    toks = b"".join(_str(f"t{i}") for i in range(hp["n_vocab"]))
    kvs.append(_str("tokenizer.ggml.tokens") + struct.pack("<IIQ", KV_ARRAY, KV_STRING, hp["n_vocab"]) + toks)
    infos, off = [], 0
    for name, ne, t, _ in plan:
        infos.append(_str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) +
                     struct.pack("<IQ", t, off))
        off = _align(off + _nbytes(ne, t))
    head = b"GGUF" + struct.pack("<IQQ", 3, len(plan), len(kvs)) + b"".join(kvs) + b"".join(infos)
    head += b"\0" * (_align(len(head)) - len(head))
    sha = hashlib.sha256()
    tmp = path + ".part"
    with open(tmp, "wb") as f:
        def put(b):
            f.write(b)
            sha.update(b)
        put(head)
        pos = 0
        for ti, (name, ne, t, init) in enumerate(plan):
            n = int(np.prod(ne))
            if init == "ones":
                put(np.ones(n, dtype=np.float32).tobytes())
            else:
                step = chunk - chunk % 32
                for s in range(0, n, step):
                    x = normal_chunk(seed, ti, s, min(step, n - s))
                    if t == T_Q8_0:
                        put(quantize_q8_0(x).tobytes())
                    elif t == T_F16:
                        put(x.astype(np.float16).tobytes())
                    else:
                        put(x.tobytes())
            nb = _nbytes(ne, t)
            pad = _align(pos + nb) - (pos + nb)
            put(b"\0" * pad)
            pos += nb + pad
    os.replace(tmp, path)
    return sha.hexdigest()


def main(argv=None):
    import argparse
    ap = argparse.ArgumentParser(description="write a random-init Qwen2.5-0.5B-shaped Q8_0 GGUF")
    ap.add_argument("path")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--prompt-ids", help="also write this many seeded prompt ids to PATH.ids.txt",
                    type=int, default=0)
    a = ap.parse_args(argv)
    print(write_qwen2_q8_0(a.path, a.seed))
    if a.prompt_ids:
        with open(a.path + ".ids.txt", "w") as f:
            f.write(" ".join(str(i) for i in prompt_ids(a.seed, a.prompt_ids, QWEN2_05B["n_vocab"])) + "\n")


if __name__ == "__main__":
    main()
