"""The reference's own tiny-model fixtures (copied data, tests/golden/tiny_qwen2/,
from the reference's tests/fixtures by tests/golden/copy_tiny_qwen2_fixtures.py):
the copies are intact, and the reference CLI compiled here from its sources
(oracle/_ref/mini_infer) reproduces both stage1 goldens bit for bit -- the
bar the device hook is held to in tests/test_hook_executor_gpu.py.
"""
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FX = os.path.join(ROOT, "tests", "golden", "tiny_qwen2")
PLAIN = os.path.join(ROOT, "oracle", "_ref", "mini_infer")
NAMES = ("embd", "layer_0", "layer_1", "output_norm", "logits")


def test_fixture_copies_are_intact():
    man = json.load(open(os.path.join(FX, "manifest.json")))["sha256"]
    assert "tiny_qwen2.gguf" in man and "tiny_qwen2_q8_0.gguf" in man and len(man) == 22
    for f, h in man.items():
        assert hashlib.sha256(open(os.path.join(FX, f), "rb").read()).hexdigest() == h, f


def dump_and_compare(exe, tmp_path, env=None):
    """Runs exe's --dump for the prefill (ids 0..4) and the decode (id 5 at
    n_past 5) goldens; returns the stderr of both runs. Asserts bitwise equality."""
    errs = []
    for golden, ids, extra in (("stage1_golden_prefill", "0 1 2 3 4", []),
                               ("stage1_golden_decode", "0 1 2 3 4 5", ["--dump-n-past", "5"])):
        d = tmp_path / golden
        d.mkdir()
        idf = tmp_path / (golden + ".ids")
        idf.write_text(ids)
        r = subprocess.run([exe, os.path.join(FX, "tiny_qwen2.gguf"), "--prompt-ids", str(idf), "-c", "16",
                            "--dump", str(d)] + extra, capture_output=True, text=True, timeout=120, env=env)
        assert r.returncode == 0, r.stderr[-2000:]
        errs.append(r.stderr)
        for n in NAMES:
            got = open(d / (n + ".bin"), "rb").read()
            want = open(os.path.join(FX, golden, n + ".bin"), "rb").read()
            assert open(d / (n + ".shape")).read() == open(os.path.join(FX, golden, n + ".shape")).read()
            if got != want:
                a = np.frombuffer(got, np.float32)
                b = np.frombuffer(want, np.float32)
                raise AssertionError(f"{golden}/{n}: {int((a != b).sum())} of {a.size} floats differ, "
                                     f"max {float(np.abs(a - b).max()):.3e}")
    return errs


def test_compiled_reference_reproduces_goldens(tmp_path):
    if not os.path.exists(PLAIN):
        pytest.skip("oracle/_ref/mini_infer is not built (the reference tree was absent)")
    dump_and_compare(PLAIN, tmp_path)


Q8_TOKENS = "3 7 1 22 5"  # tests/test_model_qwen2.cpp:248


def batch_and_incremental(exe, tmp_path, env=None):
    """Logits of the Q8_0 tiny model for Q8_TOKENS: one batched prefill call
    (--dump) and one token per call (--dump-incremental); returns both arrays
    and the stderr of the two runs."""
    idf = tmp_path / "q8.ids"
    idf.write_text(Q8_TOKENS)
    model = os.path.join(FX, "tiny_qwen2_q8_0.gguf")
    out, errs = [], []
    for flag in ("--dump", "--dump-incremental"):
        d = tmp_path / flag.strip("-")
        d.mkdir()
        r = subprocess.run([exe, model, "--prompt-ids", str(idf), "-c", "16", flag, str(d)],
                           capture_output=True, text=True, timeout=120, env=env)
        assert r.returncode == 0, r.stderr[-2000:]
        errs.append(r.stderr)
        if flag == "--dump":
            out.append(np.fromfile(d / "logits.bin", np.float32).reshape(5, -1))
        else:
            out.append(np.stack([np.fromfile(d / f"logits_step_{i}.bin", np.float32).reshape(-1)
                                 for i in range(5)]))
    return out[0], out[1], errs


def test_compiled_reference_q8_batch_equals_incremental(tmp_path):
    # tests/test_model_qwen2.cpp:241-288: zero mismatches between the batched
    # and the token-by-token logits of the Q8_0 tiny model
    if not os.path.exists(PLAIN):
        pytest.skip("oracle/_ref/mini_infer is not built (the reference tree was absent)")
    batch, incr, _ = batch_and_incremental(PLAIN, tmp_path)
    assert batch.shape == (5, 64)
    assert np.array_equal(batch.view(np.uint32), incr.view(np.uint32))
