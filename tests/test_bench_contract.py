"""bench.py on the host: its algorithmic figures and its one-GPU contract.

The roofline's `achieved` is algorithmic bytes (or FLOPs) per launch divided
by the kernel time, so the per-launch figures are pinned here to the values
computed by hand from the workload's shapes (K and V read once, Q read and O
written once per layer; 4 D FLOPs per (head, query, visible key)):
- decode, 24 layers x n_kv 4096, 14 Q / 2 KV heads, D 64, F32:
  24 (2 * 4096 * 2 * 64 * 4 + 2 * 14 * 64 * 4) = 100,835,328 bytes;
- one layer at n_kv 512: 531,456 bytes;
- the 7B shape (28 / 4 heads, D 128, F16 cache, n_kv 8192): 16,805,888 bytes;
- causal prefill at n = 1024 and 4096 (14 heads, D 64): 1,880,883,200 and
  30,072,111,104 FLOPs.
"""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_decode_bytes_per_launch():
    assert bench.decode_bytes(24, 4096, 14, 2, 64, 4) == 100_835_328
    assert bench.decode_bytes(1, 512, 14, 2, 64, 4) == 531_456
    assert bench.decode_bytes(1, 8192, 28, 4, 128, 2) == 16_805_888
    # the sweep's sizes scale as 1024 n_kv + 7168 bytes per layer
    for n_kv in (128, 1024, 16384, 32768):
        assert bench.decode_bytes(24, n_kv, 14, 2, 64, 4) == 24 * (1024 * n_kv + 7168)


def test_causal_prefill_flops():
    assert bench.causal_flops(1024, 14, 64) == 1_880_883_200
    assert bench.causal_flops(4096, 14, 64) == 30_072_111_104
    # one query seeing one key: QK and PV, 2 D multiply-adds each
    assert bench.causal_flops(1, 1, 64) == 4 * 64


def test_peaks_are_the_published_ones():
    assert bench.HBM_PEAK_GBPS == 8000.0
    assert bench.FP32_MFMA_PEAK_TFLOPS == 157.3
    assert bench.BF16_MFMA_PEAK_TFLOPS == 2500.0


def test_more_than_one_gpu_is_refused_before_any_gpu_work():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""
