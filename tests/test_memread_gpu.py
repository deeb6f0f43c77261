"""The read-bandwidth ceiling pass (mi_hip_memread, the device counterpart of
tools/bench_memread.cpp): every workgroup's sum is its slice's sum, so every
byte of the buffer was read once and accumulated."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def slice_sums(x, n_sums):
    """float64 sums of the workgroup slices (16-byte pieces split as the kernel does)."""
    n4 = x.size // 4
    per = -(-n4 // n_sums)
    return np.array([x[4 * w * per:4 * min((w + 1) * per, n4)].astype(np.float64).sum()
                     for w in range(n_sums)])


@pytest.mark.parametrize("n_floats,n_sums", [(4, 1), (4 * 1000 + 8, 7), (1 << 20, 256),
                                             ((1 << 22) + 36, 1000), (64, 65536)])
def test_slice_sums(hip, stream, n_floats, n_sums):
    import torch
    print(f"memread n_floats={n_floats} n_sums={n_sums}", flush=True)
    g = torch.Generator().manual_seed(n_floats + n_sums)
    x = torch.rand(n_floats, generator=g, dtype=torch.float32)
    dx = x.cuda()
    sums = torch.full((n_sums,), float("nan"), device="cuda")
    hip.check(hip.mi_hip_memread(ctypes.c_void_p(dx.data_ptr()), n_floats * 4,
                                 ctypes.c_void_p(sums.data_ptr()), n_sums, stream))
    torch.cuda.synchronize()
    got = sums.cpu().numpy().astype(np.float64)
    want = slice_sums(x.numpy(), n_sums)
    # float32 partial sums of at most ~4M uniform [0, 1) values
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-4)
