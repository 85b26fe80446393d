"""The moe_ffn_cuda-signature C++ shim (include/ember_moe_compat.hpp) through a native HIP program
that follows the reference's tools/moe_ffn_test.cu procedure (double reference, max |err| < 1e-4)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "native", "moe_ffn_compat_test")

pytestmark = pytest.mark.gpu


def test_compat_shim_against_double_reference(gpu):
    assert os.path.exists(EXE), "build with __graft_entry__.build()"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("all ok")
