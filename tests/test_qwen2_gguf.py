"""CPU checks of the model-file generator (qwen2_gguf.py) and of the engine's
GGUF loader error paths (no GPU needed: mi_hip_qwen2_load validates the file
before it touches a device).

The generator is pinned three ways: its Q8_0 quantiser is bit-identical to the
reference's (src/quant.cpp:129-153, via oracle/_ref), its files load and run in
the reference engine itself (oracle/_ref/mini_infer, src/gguf.cpp:259-436 and
src/model_qwen2.cpp:426-537), and its output bytes are pinned by sha256."""
import ctypes
import hashlib
import os
import struct
import subprocess

import numpy as np
import pytest

import mi_hip_attn as mh
import qwen2_gguf as gg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MINI_INFER = os.path.join(ROOT, "oracle", "_ref", "mini_infer")

TINY = dict(n_vocab=512, n_embd=128, n_layer=2, n_head=2, n_head_kv=1, n_ff=256,
            n_ctx_train=4096, rope_freq_base=10000.0, rms_eps=1e-6)
# sha256 of write_qwen2_q8_0(path, 7, TINY): any change to the generator, the
# quantiser or the file layout changes it (and the 0.5B fixture's pin).
TINY_SHA = "7ecc5fd6d970643d26c02d1719da4a9f7724e23302df821db30f3e614bf0ce5f"


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("gguf") / "tiny.gguf")
    sha = gg.write_qwen2_q8_0(path, 7, TINY)
    return path, sha


def test_splitmix64_known_answers():
    # splitmix64's published first outputs for state 0 (the generator adds the
    # golden gamma before mixing, as the reference algorithm does).
    z = np.array([0], dtype=np.uint64)
    out = []
    for _ in range(3):
        out.append(int(gg.splitmix64(z)[0]))
        z = z + gg._GOLD
    assert out == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_normal_draws_are_deterministic_and_chunk_independent():
    a = gg.normal_chunk(5, 3, 0, 4096)
    b = np.concatenate([gg.normal_chunk(5, 3, 0, 1000), gg.normal_chunk(5, 3, 1000, 3096)])
    assert np.array_equal(a, b)
    assert not np.array_equal(a, gg.normal_chunk(5, 4, 0, 4096))  # tensors differ
    assert not np.array_equal(a, gg.normal_chunk(6, 3, 0, 4096))  # seeds differ


def test_normal_draws_statistics():
    x = gg.normal_chunk(1, 0, 0, 1 << 20).astype(np.float64)
    assert abs(x.mean()) < 1e-4
    assert abs(x.std() - 0.02) < 2e-4
    # Irwin-Hall(4): bounded at 2 * sqrt(3) standard deviations, kurtosis 3 - 6 / 20 = 2.7
    assert np.abs(x).max() <= 0.02 * 2 * np.sqrt(3) * (1 + 1e-6)
    k = ((x - x.mean()) ** 4).mean() / x.var() ** 2
    assert abs(k - 2.7) < 0.02


def test_quantizer_matches_reference():
    from oracle import cpu_attention
    ref = cpu_attention.reference()
    if ref is None:
        pytest.skip("oracle/_ref is not built")
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 257) * 0.02).astype(np.float32)
    x[:32] = 0.0                                            # all-zero block
    x[32:64] = np.arange(-16, 16, dtype=np.float32) / 127   # amax 16/127: scale 16/127^2
    x[64:96] = np.float32(1e-30) * rng.standard_normal(32).astype(np.float32)  # fp16 scale underflows
    fn = ref.lib.ref_quantize_rows_q8_0
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
    want = np.empty(x.size // 32 * 34, np.uint8)
    fn(x.ctypes.data, want.ctypes.data, x.size, 1)
    got = gg.quantize_q8_0(x)
    assert got.tobytes() == want.tobytes()


def test_prompt_ids_in_range_and_seeded():
    ids = gg.prompt_ids(1234, 128, 151936)
    assert len(ids) == 128 and min(ids) >= 0 and max(ids) < 151936
    assert ids == gg.prompt_ids(1234, 128, 151936) and ids != gg.prompt_ids(1235, 128, 151936)


def test_file_layout(tiny):
    path, sha = tiny
    data = open(path, "rb").read()
    assert hashlib.sha256(data).hexdigest() == sha
    assert data[:4] == b"GGUF" and struct.unpack("<I", data[4:8])[0] == 3
    n_t, n_kv = struct.unpack("<QQ", data[8:24])
    assert n_t == 2 + 12 * TINY["n_layer"] and n_kv == 11
    assert sha == TINY_SHA


def test_reference_engine_runs_the_file(tiny, tmp_path):
    if not os.path.exists(MINI_INFER):
        pytest.skip("oracle/_ref/mini_infer is not built")
    path, _ = tiny
    ids = tmp_path / "ids.txt"
    ids.write_text(" ".join(map(str, gg.prompt_ids(7, 9, TINY["n_vocab"]))))
    r = subprocess.run([MINI_INFER, path, "--prompt-ids", str(ids), "-c", "64", "-n", "12", "-t", "1"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = [int(t) for t in r.stdout.split()]
    assert len(out) == 12 and all(0 <= t < TINY["n_vocab"] for t in out)


def load_status(lib, path):
    h = ctypes.c_void_p()
    rc = lib.mi_hip_qwen2_load(os.fsencode(path), 64, 0, ctypes.byref(h))
    return rc, lib.last_error(), h.value


def test_loader_rejects_bad_files(tiny, tmp_path):
    lib = mh.lib()
    rc, msg, h = load_status(lib, str(tmp_path / "missing.gguf"))
    assert rc == 1 and "cannot open" in msg and h is None
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUF" + struct.pack("<IQQ", 2, 0, 0))
    rc, msg, _ = load_status(lib, str(bad))
    assert rc == 1 and "version" in msg
    bad.write_bytes(b"NOPE" + bytes(20))
    rc, msg, _ = load_status(lib, str(bad))
    assert rc == 1 and "magic" in msg
    data = open(tiny[0], "rb").read()
    bad.write_bytes(data[: len(data) // 2])  # tensor data cut short
    rc, msg, _ = load_status(lib, str(bad))
    assert rc == 1 and "past end of file" in msg


def test_loader_accepts_the_generated_file_up_to_the_device(tiny):
    # The file validates; with no device initialised the load stops at the first
    # device step with a state error, not a format error.
    lib = mh.lib()
    if lib.mi_hip_init(0) == 0:
        pytest.skip("a device is present: covered by the GPU tests")
    rc, msg, _ = load_status(lib, tiny[0])
    assert rc == 6 and "mi_hip_init" in msg, msg
