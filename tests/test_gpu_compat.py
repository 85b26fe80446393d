"""The moe_ffn_cuda-signature C++ shim (include/ember_moe_compat.hpp) through a native HIP program,
tests/native/compat_shim_check.cpp: F32 layers at the 1e-4 / 1e-5 bar and a Q8_0 layer at 2e-3
against the CPU oracle, and a captured HIP graph of the decode call replayed on fresh inputs (bit-equal
to the eager call, within the bar of the oracle)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "native", "compat_shim_check")
ORACLE = os.path.join(ROOT, "oracle", "liboracle.so")

pytestmark = pytest.mark.gpu


def test_compat_shim_against_oracle(gpu):
    assert os.path.exists(EXE), "build with __graft_entry__.build()"
    assert os.path.exists(ORACLE), "build with __graft_entry__.build()"
    r = subprocess.run([EXE, ORACLE], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("all ok")
    assert r.stdout.count("graph replay") == 6
