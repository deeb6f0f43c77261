"""Pins the CPU oracle (oracle/attn_oracle.cpp) before anything is compared to it.

1. Golden vectors: outputs of the reference's own ops (compiled in place from
   src/ops_cpu.cpp etc., see tests/golden/make_golden.py) -- bit-exact, at
   several thread counts (the static split of src/ops_cpu.cpp:46-53 never
   changes a result).
2. Mathematics the reference's output is fixed by, chosen so that a plausible
   slip (wrong GQA index, transposed operand, off-by-one mask, missing scale)
   fails: float64 brute force, one-hot known answers, invariants.
3. The reference's own known-answer softmax test (tests/test_ops_cpu.cpp:215-241)
   and rope tests (tests/test_ops_cpu.cpp:181-213).
"""
import numpy as np
import pytest

from conftest import case_inputs, load_golden
from oracle import cpu_attention


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def f16_cache(k, v):
    return (cpu_attention.fp16_widen(k.astype(np.float16)),
            cpu_attention.fp16_widen(v.astype(np.float16)))


@pytest.mark.parametrize("n_threads", [1, 3, 8])
def test_oracle_matches_reference_goldens_bitwise(oracle, golden_manifest, n_threads):
    for name, c in golden_manifest["cases"].items():
        q, k, v = case_inputs(c)
        if c["kv_type"] == "f16":
            k, v = f16_cache(k, v)
        scores, probs, out = oracle.attention(q, k, v, c["n_past"], c["scale"], n_threads)
        g = load_golden(name)
        assert np.array_equal(bits(out), bits(g["out"])), name
        if "scores" in g:
            assert np.array_equal(bits(scores), bits(g["scores"])), name
            assert np.array_equal(bits(probs), bits(g["probs"])), name


def test_golden_files_are_what_the_manifest_recorded(golden_manifest):
    for name, c in golden_manifest["cases"].items():
        g = load_golden(name)
        for key, digest in c["sha256"].items():
            assert cpu_attention.sha256(g[key]) == digest, (name, key)


def test_softmax_known_answer_from_reference_tests(oracle):
    # tests/test_ops_cpu.cpp:215-241: [n_kv=4, n_tokens=2], masked 99s never leak.
    import ctypes
    from mi_hip_attn import make_tensor, MI_OP_SOFTMAX
    src = np.array([5, 99, 99, 99, 1, 3, 99, 99], np.float32)
    dst = np.full(8, np.nan, np.float32)
    s = make_tensor(src.ctypes.data, [4, 2, 1], [4, 16, 32])
    d = make_tensor(dst.ctypes.data, [4, 2, 1], [4, 16, 32], op=MI_OP_SOFTMAX, src=[s],
                    params=[0, 1.0])
    fn = oracle.lib.oracle_softmax
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    fn(ctypes.addressof(d), 0, 1)
    assert dst[0] == 1.0 and dst[1] == 0 and dst[2] == 0 and dst[3] == 0
    e0, e1 = np.exp(np.float32(-2.0)), np.float32(1.0)
    assert abs(dst[4] - e0 / (e0 + e1)) < 1e-6 and abs(dst[5] - e1 / (e0 + e1)) < 1e-6
    assert dst[6] == 0 and dst[7] == 0
    g = load_golden("softmax_kat")
    assert np.array_equal(bits(dst), bits(g["probs"].reshape(-1)))


def test_fp16_widening_is_exact_for_every_code(golden_manifest):
    codes = np.arange(65536, dtype=np.uint16)
    ours = cpu_attention.fp16_widen(codes)
    numpy_ref = codes.view(np.float16).astype(np.float32)  # IEEE widening, a library routine
    assert np.array_equal(bits(ours), bits(numpy_ref))
    # ... and the reference's own converter (src/quant.cpp:26-63) over all codes.
    assert cpu_attention.sha256(bits(ours)) == golden_manifest["fp16_lut_sha256"]


@pytest.mark.parametrize("n,nth", [(0, 1), (1, 4), (7, 3), (100, 8), (14 * 512, 16), (5, 8)])
def test_split_range_partitions_with_remainder_first(oracle, n, nth):
    spans = [oracle.split_range(n, i, nth) for i in range(nth)]
    assert spans[0][0] == 0 and spans[-1][1] == n
    for (a, b), (c, _) in zip(spans, spans[1:]):
        assert b == c
    sizes = [b - a for a, b in spans]
    assert max(sizes) - min(sizes) <= 1
    assert sizes == sorted(sizes, reverse=True)  # the extra units go to the front


def brute_force(q, k, v, n_past, scale):
    """float64 attention straight from the definitions (causal, GQA h -> h // n_rep)."""
    t, h, d = q.shape
    n_kv = n_past + t
    n_rep = h // k.shape[1]
    q64, k64, v64 = (x.astype(np.float64) for x in (q, k, v))
    scores = np.zeros((h, t, n_kv))
    probs = np.zeros((h, t, n_kv))
    out = np.zeros((t, h, d))
    for hh in range(h):
        g = hh // n_rep
        for j in range(t):
            s = k64[:n_kv, g, :] @ q64[j, hh, :]
            scores[hh, j] = s
            vis = n_past + j + 1
            x = s[:vis] * scale
            e = np.exp(x - x.max())
            probs[hh, j, :vis] = e / e.sum()
            out[j, hh] = probs[hh, j] @ v64[:n_kv, g, :]
    return scores, probs, out


@pytest.mark.parametrize("shape", [
    # head_dim, n_head, n_head_kv, n_ctx, n_past, n_tokens
    (4, 2, 1, 9, 0, 5),
    (64, 14, 2, 40, 3, 6),
    (64, 14, 2, 80, 79, 1),
    (128, 8, 2, 30, 0, 17),
    (32, 6, 3, 12, 4, 4),
])
def test_oracle_matches_float64_definition(oracle, shape):
    d, h, hkv, n_ctx, n_past, t = shape
    q, k, v = cpu_attention.make_inputs(99 + d + h, d, h, hkv, n_ctx, t)
    scale = float(np.float32(1) / np.sqrt(np.float32(d)))
    s, p, o = oracle.attention(q, k, v, n_past, scale, 2)
    s64, p64, o64 = brute_force(q, k, v, n_past, scale)
    assert np.allclose(s, s64, rtol=1e-5, atol=1e-5)
    assert np.allclose(p, p64, rtol=1e-5, atol=1e-6)
    assert np.allclose(o, o64, rtol=1e-5, atol=1e-5)


def test_brute_force_check_catches_planted_mistakes(oracle):
    # The comparison above must fail for the classic slips: a wrong GQA index
    # (h % n_hkv instead of h // n_rep) and an off-by-one causal boundary.
    d, h, hkv, n_ctx, n_past, t = 16, 4, 2, 12, 2, 5
    q, k, v = cpu_attention.make_inputs(7, d, h, hkv, n_ctx, t)
    scale = 0.25
    s, p, o = oracle.attention(q, k, v, n_past, scale, 1)
    s64, p64, o64 = brute_force(q, k, v, n_past, scale)
    wrong_gqa = s.copy()
    for hh in range(h):
        wrong_gqa[hh] = (k[: n_past + t, hh % hkv, :] @ q[:, hh, :].T).T
    assert not np.allclose(wrong_gqa, s64, rtol=1e-5, atol=1e-5)
    shifted = np.roll(p, 1, axis=2)  # mask one key too late
    assert not np.allclose(shifted, p64, rtol=1e-5, atol=1e-6)
    # A dropped term (the last head dimension left out of the dot product).
    dropped = s.copy()
    for hh in range(h):
        dropped[hh] = (k[: n_past + t, hh // (h // hkv), : d - 1] @ q[:, hh, : d - 1].T).T
    assert not np.allclose(dropped, s64, rtol=1e-5, atol=1e-5)
    # P.V with the probabilities of the wrong query row (an index slip in j).
    wrong_row = o.copy()
    for hh in range(h):
        pv = p64[hh, np.r_[1:t, 0], :]  # row j uses query j+1's probabilities
        wrong_row[:, hh, :] = pv @ v[: n_past + t, hh // (h // hkv), :].astype(np.float64)
    assert not np.allclose(wrong_row, o64, rtol=1e-5, atol=1e-5)
    assert np.allclose(o, o64, rtol=1e-5, atol=1e-5)


def test_invariants(oracle):
    d, h, hkv, n_ctx = 64, 14, 2, 48
    n_rep = h // hkv
    q, k, v = cpu_attention.make_inputs(5, d, h, hkv, n_ctx, 8)
    scale = 0.125
    # One-hot query e_3 returns K's column 3 exactly (scores are plain sums).
    q1 = np.zeros_like(q)
    q1[:, :, 3] = 1.0
    s, p, o = oracle.attention(q1, k, v, 40, scale, 1)
    for hh in range(h):
        assert np.array_equal(s[hh, 0], k[:48, hh // n_rep, 3])
    # Identical queries in one GQA group give identical scores.
    q2 = q.copy()
    q2[:, 1:n_rep, :] = q2[:, :1, :]
    s, p, o = oracle.attention(q2, k, v, 40, scale, 1)
    for hh in range(1, n_rep):
        assert np.array_equal(s[hh], s[0])
    # Rows sum to one, masked tail exactly zero, decode never masks.
    s, p, o = oracle.attention(q, k, v, 40, scale, 1)
    assert np.allclose(p.sum(axis=2), 1.0, atol=1e-6)
    for j in range(8):
        assert np.all(p[:, j, 40 + j + 1:] == 0.0)
    s, p, o = oracle.attention(q[:1], k, v, 47, scale, 1)
    assert np.all(p > 0)
    # A single visible key gives probability exactly 1 and the V row exactly.
    s, p, o = oracle.attention(q[:1], k, v, 0, scale, 1)
    assert np.all(p == 1.0)
    for hh in range(h):
        assert np.array_equal(o[0, hh], v[0, hh // n_rep])
    # Identical keys give uniform probabilities 1/N and the mean of the V rows.
    k_same = np.broadcast_to(k[:1], k.shape).copy()
    s, p, o = oracle.attention(q[:1], k_same, v, 47, scale, 1)
    assert np.all(p == p[0, 0, 0]) and abs(p[0, 0, 0] - 1.0 / 48) < 1e-9
    for hh in range(h):
        assert np.allclose(o[0, hh], v[:48, hh // n_rep].astype(np.float64).mean(axis=0),
                           rtol=1e-5, atol=1e-6)
    # Permuting cached positions permutes the scores (decode).
    perm = np.random.default_rng(1).permutation(48)
    s0, _, o0 = oracle.attention(q[:1], k, v, 47, scale, 1)
    s1, _, o1 = oracle.attention(q[:1], k[perm], v[perm], 47, scale, 1)
    assert np.array_equal(s1, s0[:, :, perm])
    assert np.allclose(o1, o0, atol=1e-6)
    # Scale enters only through the softmax: scores ignore it, probabilities
    # at scale s equal the probabilities of the scores pre-multiplied by s.
    s_a, p_a, _ = oracle.attention(q[:1], k, v, 47, 0.5, 1)
    s_b, p_b, _ = oracle.attention(q[:1] * np.float32(0.5), k, v, 47, 1.0, 1)
    s_c, _, _ = oracle.attention(q[:1], k, v, 47, 2.0, 1)
    assert np.array_equal(s_a, s_c)
    assert np.allclose(p_a, p_b, rtol=1e-5, atol=1e-7)


# ---- MI_OP_ROPE (src/ops_cpu.cpp:270-302) -----------------------------------

def test_rope_matches_reference_goldens_bitwise(oracle, golden_manifest):
    for name, c in golden_manifest["rope"].items():
        g = load_golden(name)
        assert cpu_attention.sha256(g["src"]) == c["sha256_src"], name
        assert cpu_attention.sha256(g["dst"]) == c["sha256_dst"], name
        y = oracle.rope(g["src"], c["n_past"], c["n_dims"], c["freq_base"])
        assert np.array_equal(bits(y), bits(g["dst"])), name


def test_rope_known_answers_from_reference_tests(oracle):
    # test_ops_cpu.cpp:181-196: position 0 is the identity for every pair.
    x = np.array([[[1, 2, 3, 4]]], np.float32)
    assert np.array_equal(oracle.rope(x, 0, 4, 10000.0), x)
    # test_ops_cpu.cpp:198-213: one pair, frequency base^0 = 1, position 5.
    y = oracle.rope(np.array([[[1, 0]]], np.float32), 5, 2, 10000.0)
    assert abs(y[0, 0, 0] - np.cos(5.0)) < 1e-6 and abs(y[0, 0, 1] - np.sin(5.0)) < 1e-6


def test_rope_pairs_halves_with_the_stated_frequencies(oracle):
    # One-hot inputs: element p may only move to p + n_dims/2 (NEOX halves, not
    # adjacent elements), by the angle pos * base^(-2p / n_dims) (float64 here).
    d, n_dims, base, pos = 64, 48, 10000.0, 3
    half = n_dims // 2
    for p in (0, 1, 7, half - 1):
        x = np.zeros((1, 1, d), np.float32)
        x[0, 0, p] = 1.0
        y = oracle.rope(x, pos, n_dims, base)[0, 0]
        theta = pos * base ** (-2.0 * p / n_dims)
        want = np.zeros(d)
        want[p], want[p + half] = np.cos(theta), np.sin(theta)
        assert np.abs(y - want).max() < 2e-6, p
        x[0, 0, p] = 0.0
        x[0, 0, p + half] = 1.0  # the partner turns the other way
        y = oracle.rope(x, pos, n_dims, base)[0, 0]
        want = np.zeros(d)
        want[p], want[p + half] = -np.sin(theta), np.cos(theta)
        assert np.abs(y - want).max() < 2e-6, p
    # elements from n_dims on pass through unchanged
    x = np.random.default_rng(3).standard_normal((2, 3, d)).astype(np.float32)
    y = oracle.rope(x, 17, n_dims, base)
    assert np.array_equal(y[..., n_dims:], x[..., n_dims:])


def test_rope_rotations_keep_pair_norms_and_compose(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 3, 64)).astype(np.float32)
    y = oracle.rope(x, 100, 64, 1000000.0)
    n0 = np.hypot(x[..., :32].astype(np.float64), x[..., 32:])
    n1 = np.hypot(y[..., :32].astype(np.float64), y[..., 32:])
    assert np.abs(n1 - n0).max() < 1e-5 * max(1.0, n0.max())
    # token t of a call at n_past is position n_past + t: one call over four
    # tokens equals four one-token calls
    for t in range(4):
        one = oracle.rope(x[t:t + 1], 100 + t, 64, 1000000.0)
        assert np.array_equal(bits(one[0]), bits(y[t]))


def test_rope_oracle_equals_reference_library(oracle):
    ref = cpu_attention.reference()
    if ref is None:
        pytest.skip("oracle/_ref (the reference compiled in place) is not built")
    import ctypes
    fn = ref.lib.ref_rope
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 5 + [ctypes.c_float]
    rng = np.random.default_rng(6)
    for (d, h, t, n_past, n_dims, base) in [(64, 14, 9, 4000, 64, 1e6), (128, 4, 3, 65000, 128, 1e6),
                                            (64, 2, 5, 0, 16, 500.0), (8, 3, 2, 7, 6, 10000.0)]:
        x = rng.standard_normal((t, h, d)).astype(np.float32)
        want = np.empty_like(x)
        fn(x.ctypes.data, want.ctypes.data, d, h, t, n_past, n_dims, ctypes.c_float(base))
        assert np.array_equal(bits(oracle.rope(x, n_past, n_dims, base)), bits(want))


# ---- Q8_0: MI_OP_QUANTIZE_Q8_0 and MI_OP_MUL_MAT with Q8_0 weights -----------

def test_q8_0_matches_reference_goldens_bitwise(oracle, golden_manifest):
    for name, c in golden_manifest["q8_0"].items():
        g = load_golden(name)
        for key in ("w", "x", "act", "dst"):
            assert cpu_attention.sha256(g[key]) == c["sha256_" + key], (name, key)
        act = oracle.quantize_q8_0_act(g["x"])
        assert np.array_equal(act, g["act"]), name
        dst = oracle.mul_mat_q8_0(g["w"], g["act"], c["k"], c["n"], c["m"])
        assert np.array_equal(bits(dst), bits(g["dst"])), name


def test_q8_0_activation_known_answers(oracle):
    # all-zero block -> scale 0, values 0; amax 127 -> scale exactly 1, and
    # x.5 values round half to even (lrintf); |q| never passes 127
    x = np.zeros((1, 64), np.float32)
    x[0, 32:] = np.arange(32, dtype=np.float32) - 15.5
    x[0, 63] = 127.0
    d, q = cpu_attention.q8_act_blocks(oracle.quantize_q8_0_act(x), 1, 64)
    assert d[0, 0] == 0 and not q[0, 0].any()
    assert d[0, 1] == np.float32(1.0)
    want = np.rint(x[0, 32:]).astype(np.int64)  # numpy rint: half to even
    want[-1] = 127
    assert np.array_equal(q[0, 1].astype(np.int64), want)
    y = np.random.default_rng(9).standard_normal((3, 96)).astype(np.float32) * 50
    d, q = cpu_attention.q8_act_blocks(oracle.quantize_q8_0_act(y), 3, 96)
    amax = np.abs(y.reshape(3, 3, 32)).max(axis=2)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))
    assert np.abs(q).max() == 127 and np.all(np.abs(q.astype(np.int64)) <= 127)


def test_q8_0_dot_equals_dequantized_float64_product(oracle, golden_manifest):
    # The order-free value of the dot: sum over blocks of fp16(w.d) * a.d *
    # sum(w.qs * a.qs), in float64. A dropped scale, swapped operand or wrong
    # grouping moves the result far beyond float rounding.
    for name in golden_manifest["q8_0"]:
        c = golden_manifest["q8_0"][name]
        g = load_golden(name)
        k, n, m = c["k"], c["n"], c["m"]
        wd, wq = cpu_attention.q8_weight_blocks(g["w"], n, k)
        ad, aq = cpu_attention.q8_act_blocks(g["act"], m, k)
        isum = np.einsum("nbk,mbk->mnb", wq.astype(np.int64), aq.astype(np.int64))
        want = np.einsum("mnb,nb,mb->mn", isum.astype(np.float64), wd.astype(np.float64),
                         ad.astype(np.float64))
        got = oracle.mul_mat_q8_0(g["w"], g["act"], k, n, m)
        scale = np.abs(want).max() + 1e-12
        assert np.abs(got - want).max() <= 1e-5 * scale, name
