"""CPU check of the kernels' temperature division (tests/cpp/div_check.c).

The kernels divide z by T with Markstein's FMA-corrected quotient on slices
whose logits all lie in its covered range, and with a correctly rounded
division elsewhere (zdiv in mlxforge_amd/csrc/sampler_impl.hpp).  The
reference divides once, correctly rounded (src/sample/sampler.cpp:158).  This
checks the method bit for bit against the C division: exhaustively over bf16,
over every fifth f16 temperature, and on 40 M random fp32 pairs.  The GPU
parity tests check the kernels' own arithmetic against the oracle.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cpp", "div_check.c")


def _build(tmp_path, *defs):
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not found")
    exe = str(tmp_path / ("div_check" + "".join(d.lower() for d in defs)))
    subprocess.run([gcc, "-O2", "-ffp-contract=off", *[f"-D{d}" for d in defs], SRC, "-o", exe,
                    "-lm", "-lpthread"], check=True, capture_output=True, text=True)
    return exe


def test_fma_corrected_division_is_correctly_rounded(tmp_path):
    exe = _build(tmp_path)
    proc = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "mismatches 0" in proc.stdout


def test_check_catches_missing_correction(tmp_path):
    exe = _build(tmp_path, "PLANT_NO_CORRECTION")
    proc = subprocess.run([exe, "50", "200000"], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 1
    bad = int(proc.stdout.split("mismatches")[-1])
    assert bad > 1000
