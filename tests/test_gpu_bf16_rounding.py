"""The FP32 -> BF16 rounding of every BF16 output (gfx950's v_cvt_pk_bf16_f32
through loom_dev::bf16x2_pack) against the reference's conversion,
half::bf16::from_f32 (round to nearest even; a NaN keeps sign and top payload
with the quiet bit set), over all 2^32 FP32 bit patterns in both halves of the
packed pair.  The check is a device program (tests/checks/bf16_rounding_check.hip, built
by tests/checks/build_checks.sh, which build() runs); it runs in well under a
second."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "tests", "checks", "bin", "bf16_rounding_check")


@pytest.mark.gpu
def test_hardware_bf16_rounding_matches_the_reference_conversion_exhaustively():
    assert os.path.exists(CHECK), "build the checks first (bash tests/checks/build_checks.sh)"
    p = subprocess.run([CHECK], capture_output=True, text=True, timeout=90)
    print(p.stdout, p.stderr, flush=True)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "4294967296 patterns, 0 mismatching pairs" in p.stdout
