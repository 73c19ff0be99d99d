"""Exhaustive CPU check of the store_int8 kernel's quotient arithmetic over its
whole input domain (all finite bf16 row maxima x all |x| <= amax)."""
import json
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "native" / "quotient_check.c"


def _run(tmp_path, *defines):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path / ("qc" + "".join(d.strip("-") for d in defines))
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", *defines,
                    str(SRC), "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return json.loads(out)


def test_quotient_codes_exact_on_whole_domain(tmp_path):
    r = _run(tmp_path)
    assert r["pairs"] == 1065369600
    assert r["code_mismatch"] == 0
    assert r["div_mismatch_big"] == 0


def test_quotient_check_catches_missing_correction(tmp_path):
    r = _run(tmp_path, "-DPLANT_NO_CORRECTION")
    assert r["code_mismatch"] > 0
