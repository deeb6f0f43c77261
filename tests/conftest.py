import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mini-infer-llama.cpp_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import cpu_attention  # noqa: E402

# Parity bar: max-abs 1e-4 / rel 1e-4 for F32 K/V, 1e-2 for F16 K/V.
TOL_F32 = dict(atol=1e-4, rtol=1e-4)
TOL_F16 = dict(atol=1e-2, rtol=1e-2)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    return cpu_attention.oracle()


@pytest.fixture(scope="session")
def golden_manifest():
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        return json.load(f)


def load_golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def case_inputs(c):
    """Seeded inputs of a golden case, checked against the recorded sha256."""
    q, k, v = cpu_attention.make_inputs(c["seed"], c["head_dim"], c["n_head"], c["n_head_kv"],
                                        c["n_ctx"], c["n_tokens"])
    assert cpu_attention.sha256(q) == c["sha256_q"], "input generator drifted (q)"
    assert cpu_attention.sha256(k) == c["sha256_k"], "input generator drifted (k)"
    assert cpu_attention.sha256(v) == c["sha256_v"], "input generator drifted (v)"
    return q, k, v


@pytest.fixture(scope="session")
def hip():
    """The HIP library, initialised on device 0. Only for tests marked gpu.
    Every GPU test module requests it (directly or through usefixtures), so
    that torch's HIP runtime initialises the device before the library's own
    does: with the order reversed, torch.cuda.is_available() has reported no
    device in the same process."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import mi_hip_attn
    lib = mi_hip_attn.lib()  # raises if the library is not built
    lib.init(0)
    return lib


@pytest.fixture()
def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream
