"""bench.py's host-side logic, on the CPU: the one-GPU rule, the algorithmic bytes the roofline divides
by, the last-level-cache copy rule, and the lookup of the committed traffic summaries (a layer re-encoded
with --expert-type never borrows the config's own figure)."""
import os
import subprocess
import sys

import pytest

import ember_moe as em

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_slice_launch_bytes_c2_t1():
    # Mixtral-shaped Q8_0 layer, one token, two experts hit, on the slice path: gate, up and down of both
    # picks in Q8_0 (34 bytes per 32 weights), the 2 x 224 partial rows of 4096 floats, the token and the
    # F32 router
    spec = bench.layer_spec("c2")
    gu, layer, flops = bench.algorithmic(spec, 1, 2, em.PATH_SLICES)
    w = 2 * 3 * 4096 * 14336 * 34 // 32
    assert gu == w + 2 * 224 * 4096 * 4 + 4096 * 4 + 8 * 4096 * 4 == 381829120
    assert layer == w + 8 * 4096 * 4 + 2 * 4096 * 4
    assert flops == 2.0 * (2 * 3 * 4096 * 14336) + 2.0 * 8 * 4096


def test_gate_up_bytes_without_slices():
    spec = bench.layer_spec("c3")
    T, U = 32, 100
    gu, _, _ = bench.algorithmic(spec, T, U, 0)
    assert gu == pytest.approx(U * 2 * 2048 * 768 * 144 / 256 + T * 8 * 2048 * 4 + T * 8 * 768 * 4)


@pytest.mark.parametrize("touched,want", [(1, 16), (64 << 20, 8), (256 << 20, 2), (600 << 20, 1), (10 << 30, 1)])
def test_copies_cover_twice_the_last_level_cache(touched, want):
    n = bench.copies_needed(touched)
    assert n == want
    assert n == bench.MAX_COPIES or n * touched >= 2 * bench.LLC_BYTES


def test_traffic_lookup_is_keyed_by_workload():
    assert bench.profiled_traffic("c2", 1) == 384200000.0  # the committed C2 T = 1 summary
    assert bench.profiled_traffic("c2:q4_k", 1) is None    # re-encoded: no summary of its own
    assert bench.profiled_traffic("c2", 3) is None
