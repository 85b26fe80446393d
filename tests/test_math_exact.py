"""Pins the device math restatements (ember.cpp_amd/csrc/moe_math.hpp): the exp tables are recomputed
from their definition, and the same header compiled for the host is compared with glibc's expf
(all 2^32 inputs) and exp (a 2e7-sample sweep of [-512, 0] plus special values)."""
import os
import re
import struct
import subprocess
import tempfile
from decimal import Decimal, getcontext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "ember.cpp_amd", "csrc", "moe_math.hpp")


def _table(name):
    text = open(HDR).read()
    body = text[text.index(name):]
    body = body[body.index("{") + 1:body.index("};")]
    return [int(v, 16) for v in re.findall(r"0x([0-9a-f]+)ull", body)]


def _bits(f):
    return struct.unpack("<Q", struct.pack("<d", f))[0]


def test_tables_recomputed():
    getcontext().prec = 80
    ln2 = Decimal(2).ln()
    t32 = _table("kExp2Tab32")
    assert len(t32) == 32
    for i in range(32):
        assert t32[i] == (_bits(float((ln2 * i / 32).exp())) - (i << 47)) & (2 ** 64 - 1)
    t128 = _table("kExp2Tab128")
    assert len(t128) == 256
    for k in range(128):
        v = (ln2 * k / 128).exp()
        s = float(v)
        assert t128[2 * k] == _bits(float((v - Decimal(s)) / Decimal(s)))
        assert t128[2 * k + 1] == (_bits(s) - (k << 45)) & (2 ** 64 - 1)


PROG = r"""
#include "moe_math.hpp"
#include <cmath>
#include <cstdio>
int main() {
  long bad_f = 0, bad_d = 0;
#pragma omp parallel for reduction(+ : bad_f)
  for (long u = 0; u < (1L << 32); ++u) {
    const float x = ember_math::as_f32((uint32_t)u);
    const float a = expf(x), b = ember_math::expf_glibc(x);
    if (ember_math::as_u32(a) != ember_math::as_u32(b) && !(std::isnan(a) && std::isnan(b))) ++bad_f;
  }
#pragma omp parallel for reduction(+ : bad_d)
  for (long i = 0; i < 20000000; ++i) {
    uint64_t s = (uint64_t)i * 0x9E3779B97F4A7C15ULL; s ^= s >> 31; s *= 0xBF58476D1CE4E5B9ULL; s ^= s >> 29;
    const double x = -((double)(s >> 11) * 0x1p-53) * ((i & 1) ? 40.0 : 512.0);
    if (ember_math::as_u64(exp(x)) != ember_math::as_u64(ember_math::exp_glibc(x))) ++bad_d;
  }
  const double sp[] = {0.0, -0.0, 1e-300, -1e-300, 0x1p-60, -0x1p-54, 1.0, -1.0, 88.5, -745.2, -1e6, 1e6};
  for (double x : sp)
    if (ember_math::as_u64(exp(x)) != ember_math::as_u64(ember_math::exp_glibc(x))) ++bad_d;
  if (ember_math::exp_glibc(-INFINITY) != 0.0 || !std::isnan(ember_math::exp_glibc(NAN))) ++bad_d;
  printf("%ld %ld\n", bad_f, bad_d);
  return 0;
}
"""


def test_exp_restatements_match_glibc():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        open(src, "w").write(PROG)
        subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-builtin", "-I",
                        os.path.dirname(HDR), src, "-o", exe, "-lm"], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True, timeout=600).stdout.split()
    assert out == ["0", "0"], out
