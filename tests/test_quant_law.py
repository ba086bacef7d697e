"""The INT8 quantiser's division-free law (Markstein quotient plus a
just-below-half rounding offset, imfvideo_amd/csrc/quant_route.hip) equals the
reference's round_half_away(x / s) (models/sla2_vendor/kernel_sparse_qat.py:
136-141) for 16-bit inputs.  tests/quant_law_check.c enumerates the pairs; here
it runs on a stride of the tile maxima (every x for each), the full sweep being
`quant_law_check 1`."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_quant_law_matches_ieee_division(tmp_path):
    exe = str(tmp_path / "quant_law_check")
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", os.path.join(HERE, "quant_law_check.c"),
                    "-o", exe, "-lm"], check=True)
    # stride 17 reaches tile maxima whose fp16 x give the quotient 0.5 - 2^-25,
    # which a plain +0.5 offset rounds to 1 (2 mismatches at this stride)
    res = subprocess.run([exe, "17"], stdout=subprocess.PIPE, text=True, timeout=600)
    assert res.returncode == 0, res.stdout
    assert "mismatches 0" in res.stdout
