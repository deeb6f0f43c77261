"""Build-level checks of the generated gfx950 code (CPU only; hipcc cross-compiles).

The decode kernel issues its DPP multiply-adds as inline asm, which the
compiler's hazard recognizer does not look into. check_dpp_hazards.py walks the
final assembly and reports any DPP instruction that reads a VGPR written by a
VALU instruction fewer than two wait states before it. The checker itself is
pinned by planted cases.
"""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mini-infer-llama.cpp_amd")
CHECKER = os.path.join(PKG, "check_dpp_hazards.py")

sys.path.insert(0, PKG)
import check_dpp_hazards as chk  # noqa: E402


def _findings(tmp_path, body):
    path = tmp_path / "k.s"
    path.write_text("kernel:\n" + body)
    out = []
    for name, items in chk.parse_functions(str(path)).items():
        out += chk.check_function(name, items)
    return out


def test_checker_flags_a_planted_hazard(tmp_path):
    body = ("\tv_add_f32_e32 v5, v1, v2\n"
            "\tv_fmac_f32_dpp v7, v5, v9 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
            "\ts_endpgm\n")
    assert len(_findings(tmp_path, body)) == 1


def test_checker_flags_the_accumulator_too(tmp_path):
    # v_fmac reads its destination: a VALU write of the accumulator counts
    body = ("\tv_mul_f32_e32 v7, v1, v2\n"
            "\ts_nop 0\n"
            "\tv_fmac_f32_dpp v7, v5, v9 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
            "\ts_endpgm\n")
    assert len(_findings(tmp_path, body)) == 1


def test_checker_accepts_two_wait_states(tmp_path):
    body = ("\tv_add_f32_e32 v5, v1, v2\n"
            "\ts_nop 1\n"
            "\tv_fmac_f32_dpp v7, v5, v9 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
            "\ts_endpgm\n")
    assert _findings(tmp_path, body) == []


def test_checker_follows_branches_into_a_label(tmp_path):
    body = ("\tv_add_f32_e32 v5, v1, v2\n"
            "\ts_cbranch_scc1 .LBB0_2\n"
            "\ts_nop 7\n"
            ".LBB0_2:\n"
            "\tv_fmac_f32_dpp v7, v5, v9 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
            "\ts_endpgm\n")
    # the fall-through path is safe (s_nop 7); the branch path is not
    assert len(_findings(tmp_path, body)) == 1


@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs make and hipcc")
def test_generated_kernels_have_no_dpp_hazards():
    subprocess.run(["make", "-C", PKG, "asm"], check=True, capture_output=True, timeout=1200)
    asm = [os.path.join(PKG, "_build", f + ".s") for f in ("decode", "prefill")]
    r = subprocess.run([sys.executable, CHECKER, *asm], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-4000:]
    n = int(r.stdout.strip().split()[1])
    assert n > 1000, r.stdout  # the decode kernels' DPP blocks were found
