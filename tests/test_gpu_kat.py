"""The C++ known-answer driver (tests/cpp/sampler_kat.cpp) on the GPU: the
reference's tests/sample/sampler_test.cpp cases through the C++ wrapper
mlxforge_amd::Sampler, linked against the built libmlxf_sampler.so."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KAT = os.path.join(ROOT, "mlxforge_amd", "sampler_kat")


@pytest.mark.gpu
def test_cpp_known_answers():
    assert os.path.exists(KAT), "build first: python __graft_entry__.py (builds mlxforge_amd/sampler_kat)"
    proc = subprocess.run([KAT], capture_output=True, text=True, timeout=90)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "0 failed" in proc.stdout


def test_cpp_driver_is_built():
    assert os.path.exists(KAT) and os.access(KAT, os.X_OK)
