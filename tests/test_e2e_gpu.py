"""End-to-end greedy generation on the device-resident Qwen2 engine
(include/mi_hip_qwen2.h) against the reference engine itself.

Model: the random-initialised Qwen2.5-0.5B-shaped Q8_0 GGUF that
qwen2_gguf.write_qwen2_q8_0(seed) writes (regenerated here, sha256 pinned).
Reference: oracle/_ref/mini_infer (the reference CLI compiled from its own
sources). Fixtures (tests/golden/make_e2e_golden.py): 256 greedy ids after a
128-token prompt with n_ctx 2048, and the prefill call's last logits row.

Bars. With the reference-order attention (MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
every operation of a forward call is the engine's to the bit, so: the prefill
logits row is bit-identical, all 256 greedy ids are identical, a tiny model run
live through the reference binary on this host gives bit-identical logits at
every prompt position and identical ids, and token-by-token prefill equals the
batched one bit for bit (the reference's own property); this is the engine's
default mode, which test_greedy_ids_identical_to_reference runs as loaded.
With the fused kernels (attention within 1e-4) the Q8_0 activation rounding amplifies ulp
differences: logits stay within 0.1 of the reference's (|logit| <= 3.5 here;
measured 0.069) and the first token, whose top-2 margin is 0.16, is identical.
Run in lockstep with the reference-order engine under teacher forcing, the
fused engine's logits stay within 0.1 at all 256 steps and every step whose
argmax differs is a near-tie (margin within twice the logit difference); its
free-running generation is deterministic and forks from the reference's ids
only at such a step. No device allocation after load.
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

import mi_hip_attn as mh
import qwen2_gguf as gg
from qwen2 import Qwen2

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("hip")]  # torch initialises the device first

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")
MINI_INFER = os.path.join(ROOT, "oracle", "_ref", "mini_infer")
FUSED_LOGIT_TOL = 0.1
TINY = dict(n_vocab=1000, n_embd=256, n_layer=3, n_head=4, n_head_kv=2, n_ff=512,
            n_ctx_train=4096, rope_freq_base=10000.0, rms_eps=1e-6)


@pytest.fixture(scope="module")
def e2e():
    with open(os.path.join(GOLD, "e2e_qwen05_q8_0.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def model05_path(tmp_path_factory, e2e):
    path = str(tmp_path_factory.mktemp("e2e") / "qwen05_q8_0.gguf")
    print(f"writing the 0.5B model (seed {e2e['seed']})", flush=True)
    sha = gg.write_qwen2_q8_0(path, e2e["seed"])
    assert sha == e2e["model_sha256"], "the model generator's output changed"
    yield path
    os.remove(path)


@pytest.fixture(scope="module")
def model05(model05_path, e2e):
    m = Qwen2(model05_path, n_ctx=e2e["n_ctx"], max_tokens=len(e2e["prompt"]))
    yield m
    m.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_prefill_logits_bit_identical_to_reference(model05, e2e):
    model05.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
    want = np.load(os.path.join(GOLD, "e2e_qwen05_q8_0_logits.npz"))["logits_last"]
    nxt, logits = model05.forward(e2e["prompt"], n_past=0, want_logits=True)
    got = np.frombuffer(logits, dtype=np.float32)
    print(f"reference-order prefill logits: {np.count_nonzero(bits(got) != bits(want))} of "
          f"{got.size} differ, max abs {np.abs(got - want).max():.3e}")
    assert np.array_equal(bits(got), bits(want))
    assert nxt == e2e["ids"][0]


def test_greedy_ids_identical_to_reference(model05_path, e2e):
    # A model as it comes from load, in its default attention mode.
    with Qwen2(model05_path, n_ctx=e2e["n_ctx"], max_tokens=len(e2e["prompt"])) as m:
        ids = m.generate(e2e["prompt"], e2e["n_predict"])
    first_diff = next((i for i, (a, b) in enumerate(zip(ids, e2e["ids"])) if a != b), None)
    assert ids == e2e["ids"], f"first difference at step {first_diff}"


@pytest.mark.parametrize("mode", [mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER, mh.MI_HIP_QWEN2_ATTN_FUSED],
                         ids=["reference_order", "fused"])
def test_device_loop_ids_equal_per_call_loop(model05, e2e, mode):
    # mi_hip_qwen2_generate: every step's embedding reads the previous step's
    # argmax from device memory. Same ids as one forward call per token (the
    # reference's ids in reference-order mode), and no device allocation.
    model05.set_attention(mode)
    lib = model05.lib
    before = lib.alloc_stats()
    ids = model05.generate_device(e2e["prompt"], e2e["n_predict"])
    after = lib.alloc_stats()
    assert after.n_malloc == before.n_malloc
    assert model05.n_past == len(e2e["prompt"]) + e2e["n_predict"] - 1
    if mode == mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER:
        assert ids == e2e["ids"]
    else:
        assert ids == model05.generate(e2e["prompt"], e2e["n_predict"])


def test_device_loop_stops_at_n_ctx(tiny):
    # the reference's loop stops once the cache's positions are used
    # (src/main.cpp:481-484): 37 prompt positions in a 48-position cache give
    # 1 + 11 ids however many are asked for; fewer asked, fewer given
    _, path = tiny
    prompt = gg.prompt_ids(13, 37, TINY["n_vocab"])
    with Qwen2(path, n_ctx=48, max_tokens=len(prompt)) as m:
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
        per_call = m.generate(prompt, 40)
        assert len(per_call) == 12
        assert m.generate_device(prompt, 40) == per_call
        assert m.generate_device(prompt, 5) == per_call[:5]
        assert m.generate_device(prompt, 1) == per_call[:1]
        assert m.generate_device(prompt, 0) == []
        lib, h = m.lib, m.h
        out, n = (ctypes.c_int32 * 4)(), ctypes.c_int32()
        ids = (ctypes.c_int32 * 2)(5, TINY["n_vocab"])
        assert lib.mi_hip_qwen2_generate(h, ids, 2, 4, out, ctypes.byref(n)) == 1
        assert "vocabulary" in lib.last_error()
        assert lib.mi_hip_qwen2_generate(h, ids, 0, 4, out, ctypes.byref(n)) == 1
        assert lib.mi_hip_qwen2_generate(h, ids, 1, 4, None, ctypes.byref(n)) == 1


def test_one_token_step_equals_batched_bitwise(model05, e2e):
    # reference-order mode: a one-token step (its FFN's SiLU(gate) * up formed
    # in the gate/up matrix kernel's epilogue, its norms in the matrix kernels')
    # against the last row of the batched prompt (separate SiLU, norm and
    # quantize kernels) and against the reference engine's logits of that row
    model05.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
    prompt = e2e["prompt"]
    want = np.load(os.path.join(GOLD, "e2e_qwen05_q8_0_logits.npz"))["logits_last"]
    _, batched = model05.forward(prompt, n_past=0, want_logits=True)
    model05.forward(prompt[:-1], n_past=0)
    _, step = model05.forward(prompt[-1:], n_past=len(prompt) - 1, want_logits=True)
    step = np.frombuffer(step, dtype=np.float32)
    assert np.array_equal(bits(np.frombuffer(batched, dtype=np.float32)), bits(step))
    assert np.array_equal(bits(step), bits(want))


def test_fused_attention_end_to_end(model05, e2e):
    model05.set_attention(mh.MI_HIP_QWEN2_ATTN_FUSED)
    want = np.load(os.path.join(GOLD, "e2e_qwen05_q8_0_logits.npz"))["logits_last"]
    nxt, logits = model05.forward(e2e["prompt"], n_past=0, want_logits=True)
    err = np.abs(np.frombuffer(logits, dtype=np.float32) - want)
    ids = model05.generate(e2e["prompt"], e2e["n_predict"])
    agree = next((i for i, (a, b) in enumerate(zip(ids, e2e["ids"])) if a != b), len(ids))
    print(f"fused prefill logits: max abs err {err.max():.3e}; greedy ids agree for {agree} steps")
    assert err.max() <= FUSED_LOGIT_TOL
    assert nxt == e2e["ids"][0]


def test_fused_engine_in_lockstep_with_reference_order(model05, model05_path, e2e):
    # Both engines see the reference's history at every step (the prompt, then
    # the reference's ids one by one). The reference-order engine is the
    # reference engine to the bit, so its argmax is the reference's id at all
    # 256 steps. The fused engine's logits stay within 0.1 of it at every
    # step, and a step where its argmax differs is a near-tie: the reference's
    # top-1/top-2 margin there is within twice that step's logit difference.
    # The free-running fused generation is deterministic (two runs give the
    # same ids), and its first fork from the reference's ids is one of the
    # teacher-forced flips (the histories agree up to it).
    from qwen2 import fork_summary, teacher_forced
    model05.set_attention(mh.MI_HIP_QWEN2_ATTN_FUSED)
    with Qwen2(model05_path, n_ctx=e2e["n_ctx"], max_tokens=len(e2e["prompt"])) as ref:
        ref.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
        recs = teacher_forced(model05, ref, e2e["prompt"], e2e["ids"])
    assert [r["ref_id"] for r in recs] == e2e["ids"]
    worst = max(recs, key=lambda r: r["max_diff"])
    print(f"largest fused logit difference {worst['max_diff']:.4f} (step {worst['step']})", flush=True)
    assert all(r["max_diff"] <= FUSED_LOGIT_TOL for r in recs)
    flips = [r for r in recs if r["fused_id"] != r["ref_id"]]
    for r in flips:
        print(f"flip at step {r['step']}: margin {r['margin']:.4f}, logit difference {r['max_diff']:.4f}",
              flush=True)
        assert r["margin"] <= 2 * r["max_diff"]
    ids1 = model05.generate(e2e["prompt"], e2e["n_predict"])
    ids2 = model05.generate(e2e["prompt"], e2e["n_predict"])
    assert ids1 == ids2
    summ = fork_summary(recs, ids1, e2e["ids"])
    print("fork summary:", json.dumps(summ), flush=True)
    if summ["first_free_running_divergence"] is not None:
        assert summ["first_free_running_divergence"] in summ["flip_steps"]


def test_no_device_allocation_after_load(model05, e2e):
    lib = model05.lib
    before = lib.alloc_stats()
    model05.forward(e2e["prompt"][:16], n_past=0)
    for i in range(4):
        model05.forward([e2e["prompt"][16 + i]], n_past=16 + i)
    after = lib.alloc_stats()
    assert after.n_malloc == before.n_malloc and after.bytes_live == before.bytes_live


def test_forward_rejects_bad_arguments(model05, e2e):
    lib, h = model05.lib, model05.h
    nxt = ctypes.c_int32()

    def call(tokens, n_past, n=None):
        ids = (ctypes.c_int32 * max(len(tokens), 1))(*tokens)
        return lib.mi_hip_qwen2_forward(h, ids, len(tokens) if n is None else n, n_past, 1, None,
                                        ctypes.byref(nxt))
    assert call([], 0) == 1                            # no tokens
    assert call([5], 0, n=129) == 1                    # above max_tokens
    assert call([151936], 0) == 1 and "vocabulary" in lib.last_error()
    assert call([-1], 0) == 1
    assert call([5], 2048) == 1                        # past n_ctx
    assert call([5, 6], 2047) == 1
    assert call([5], 2047) == 0                        # the last position is fine


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = tmp_path_factory.mktemp("tiny")
    path = str(d / "tiny.gguf")
    gg.write_qwen2_q8_0(path, 11, TINY)
    return d, path


def test_tiny_model_all_positions_bit_identical_to_reference_engine(tiny):
    if not os.path.exists(MINI_INFER):
        pytest.skip("oracle/_ref/mini_infer is not built")
    d, path = tiny
    prompt = gg.prompt_ids(11, 37, TINY["n_vocab"])
    (d / "ids.txt").write_text(" ".join(map(str, prompt)))
    r = subprocess.run([MINI_INFER, path, "--prompt-ids", str(d / "ids.txt"), "-c", "256", "-n", "40",
                        "-t", "4"], capture_output=True, text=True, timeout=60, check=True)
    want_ids = [int(t) for t in r.stdout.split()]
    dump = d / "dump"
    dump.mkdir(exist_ok=True)
    subprocess.run([MINI_INFER, path, "--prompt-ids", str(d / "ids.txt"), "-c", "256", "--dump", str(dump)],
                   capture_output=True, timeout=60, check=True)
    rows, cols = map(int, (dump / "logits.shape").read_text().split())
    want = np.fromfile(dump / "logits.bin", dtype=np.float32).reshape(rows, cols)
    with Qwen2(path, n_ctx=256, max_tokens=len(prompt)) as m:
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
        _, logits = m.forward(prompt, n_past=0, last_logits_only=False, want_logits=True)
        got = np.frombuffer(logits, dtype=np.float32).reshape(len(prompt), TINY["n_vocab"])
        assert np.array_equal(bits(got), bits(want))
        assert m.generate(prompt, 40) == want_ids


def test_tiny_incremental_prefill_equals_batched_bitwise(tiny):
    _, path = tiny
    prompt = gg.prompt_ids(12, 24, TINY["n_vocab"])
    with Qwen2(path, n_ctx=64, max_tokens=len(prompt)) as m:
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
        _, batched = m.forward(prompt, n_past=0, want_logits=True)
        for i, t in enumerate(prompt):
            _, step = m.forward([t], n_past=i, want_logits=True)
        assert np.array_equal(bits(np.frombuffer(batched, dtype=np.float32)),
                              bits(np.frombuffer(step, dtype=np.float32)))


@pytest.mark.parametrize("head_dim,n_prompt,steps", [
    (64, 520, (511, 500, 271, 16, 3, 0)),
    (128, 300, (255, 200, 100, 40, 20, 15))])
def test_reference_order_attention_kernels_agree(tmp_path, head_dim, n_prompt, steps):
    # Reference-order attention has two kernels: rows whose V fits in LDS
    # (n_kv * head_dim * 4 <= 128 KB: n_kv <= 512 at head_dim 64, 256 at 128)
    # stage it there, longer ones read it from global memory. A batched prompt
    # longer than that takes the second for every row; one-token steps at the
    # positions in `steps` (over the cache the batched call wrote) the first,
    # with key counts that are and are not multiples of its chunks of 16, in
    # odd and even numbers of chunks. The rows' logits must agree bit for bit.
    cfg = dict(TINY, n_embd=4 * head_dim, n_ff=8 * head_dim)
    path = str(tmp_path / "m.gguf")
    gg.write_qwen2_q8_0(path, 17, cfg)
    prompt = gg.prompt_ids(5, n_prompt, cfg["n_vocab"])
    V = cfg["n_vocab"]
    with Qwen2(path, n_ctx=1024, max_tokens=len(prompt)) as m:
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
        _, rows = m.forward(prompt, n_past=0, last_logits_only=False, want_logits=True)
        rows = np.frombuffer(rows, dtype=np.float32).reshape(len(prompt), V)
        for p in steps:
            _, step = m.forward(prompt[p:p + 1], n_past=p, want_logits=True)
            assert np.array_equal(bits(rows[p]), bits(np.frombuffer(step, dtype=np.float32))), p


def test_norm_sum_walk_way_out_bitwise(tmp_path):
    # A token whose embedding row is 256 equal values (3.7): the squares' sum
    # in the reference's order rounds the same way at every step and drifts
    # more than 32 ulps from the exact prefix sums, so the 8-wave ordered sum
    # of the one-token steps' norm leaves its 64 candidates and continues the
    # chain itself (a float32 emulation of the walk takes that way out for 6
    # of the 8 segments of this row). The one-token steps must still equal the
    # batched prompt, whose norm is one lane's serial sum, bit for bit.
    seed, tok, val = 21, 5, 3.7
    path = str(tmp_path / "const_row.gguf")
    gg.write_qwen2_q8_0(path, seed, dict(TINY, embd_type=gg.T_F32))
    data = bytearray(open(path, "rb").read())
    start = bytes(data).index(gg.normal_chunk(seed, 0, 0, 4).tobytes())  # token_embd's first floats
    E = TINY["n_embd"]
    data[start + 4 * tok * E:start + 4 * (tok + 1) * E] = np.full(E, val, dtype=np.float32).tobytes()
    with open(path, "wb") as f:
        f.write(bytes(data))
    prompt = [tok, 17, tok, 3]
    with Qwen2(path, n_ctx=64, max_tokens=len(prompt)) as m:
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
        _, batched = m.forward(prompt, n_past=0, want_logits=True)
        for i, t in enumerate(prompt):
            _, step = m.forward([t], n_past=i, want_logits=True)
        assert np.array_equal(bits(np.frombuffer(batched, dtype=np.float32)),
                              bits(np.frombuffer(step, dtype=np.float32)))


@pytest.mark.parametrize("embd_type", [gg.T_F16, gg.T_F32])
def test_tiny_model_unquantised_embedding_with_separate_lm_head(tmp_path, embd_type):
    # token_embd in F16 / F32 (the embedding lookup's other types) and a separate
    # Q8_0 output.weight as the lm_head: bit-identical to the reference engine
    if not os.path.exists(MINI_INFER):
        pytest.skip("oracle/_ref/mini_infer is not built")
    hp = dict(TINY, n_layer=2, embd_type=embd_type)
    path = str(tmp_path / "m.gguf")
    gg.write_qwen2_q8_0(path, 13, hp)
    prompt = gg.prompt_ids(13, 19, hp["n_vocab"])
    (tmp_path / "ids.txt").write_text(" ".join(map(str, prompt)))
    dump = tmp_path / "dump"
    dump.mkdir()
    subprocess.run([MINI_INFER, path, "--prompt-ids", str(tmp_path / "ids.txt"), "-c", "64", "--dump",
                    str(dump)], capture_output=True, timeout=60, check=True)
    r = subprocess.run([MINI_INFER, path, "--prompt-ids", str(tmp_path / "ids.txt"), "-c", "64", "-n", "12",
                        "-t", "4"], capture_output=True, text=True, timeout=60, check=True)
    want = np.fromfile(dump / "logits.bin", dtype=np.float32).reshape(len(prompt), -1)
    with Qwen2(path, n_ctx=64, max_tokens=len(prompt)) as m:
        m.set_attention(mh.MI_HIP_QWEN2_ATTN_REFERENCE_ORDER)
        _, logits = m.forward(prompt, n_past=0, last_logits_only=False, want_logits=True)
        got = np.frombuffer(logits, dtype=np.float32).reshape(len(prompt), -1)
        assert np.array_equal(bits(got), bits(want))
        assert m.generate(prompt, 12) == [int(t) for t in r.stdout.split()]
