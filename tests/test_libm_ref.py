"""The device code's expf (csrc/libm_ref.h) against the host C library's expf,
on every one of the 2^32 float inputs (CPU: the header is compiled for the host
by g++ and run by tests/native/expf_exhaustive.cpp). The reference engine's
softmax and SiLU call that expf (src/ops_cpu.cpp:134-141, 326-331), so this is
what makes the device's values equal to the engine's bit for bit."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_ref_equals_host_expf_on_all_inputs(tmp_path):
    exe = str(tmp_path / "expf_exhaustive")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off",
                    "-I", os.path.join(ROOT, "mini-infer-llama.cpp_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "expf_exhaustive.cpp"), "-o", exe, "-lpthread"],
                   check=True)
    r = subprocess.run([exe, str(min(8, os.cpu_count() or 1))], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
