"""Operand range on the MFMA (prefill) paths, against the oracle at the 2e-3 bar.

fp16 MFMA paths (Q8_0, Q4_K, F16 stacks): activations enter as fp16 rows scaled by a power of two
(their largest magnitude in [0.5, 1)), h rows by the square of it, and the epilogues undo the scales
exactly, so activations far outside fp16's range (x ~ N(0, 1e3): h reaches ~1e6 > 65504) or deep in
its subnormals (x ~ N(0, 1e-6)) keep their precision. BF16 stacks run bf16 MFMA on the weights' own
bits with split (hi + lo) bf16 activations, so weights of 1e5 and 1e-6 (outside fp16's normal range)
are multiplied exactly. Each case also runs at one token (the GEMV path, f32 activations) and at a
batch that takes the 64- or 256-token MFMA tiles."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def _layer(spec, scales):
    """A host layer whose expert stacks are N(0, 0.02) times a per-expert factor (scales[e], cycled),
    encoded in spec.wtype."""
    s = spec
    hl = em.make_host_layer(s)

    def stack(name, rows, cols):
        v = em.normal(s.E * rows * cols, s.seed, 40 + len(name), 0.0, 0.02).reshape(s.E, rows, cols)
        v = v * np.array([scales[e % len(scales)] for e in range(s.E)], np.float32)[:, None, None]
        return em.quantize(s.wtype, np.ascontiguousarray(v, np.float32).reshape(-1))

    hl.gate = stack("gate", s.d_ff, s.d)
    hl.up = stack("up", s.d_ff, s.d)
    hl.down = stack("down_", s.d, s.d_ff)
    return hl


def _check(hl, x):
    y = run_gpu(hl, x)
    want = run_oracle(hl, x)
    assert np.all(np.isfinite(want))
    assert np.all(np.isfinite(y)), "non-finite output"
    err = rel_l2(y, want)
    print(f"  rel-L2 {err:.2e}")
    assert err < 2e-3


@pytest.mark.parametrize("wtype", [em.Q8_0, em.Q4_K, em.F16])
@pytest.mark.parametrize("xstd", [1e3, 1e-6])
@pytest.mark.parametrize("T", [1, 40, 600])
def test_fp16_paths_activation_range(gpu, wtype, xstd, T):
    spec = em.LayerSpec(d=512, d_ff=768, E=8, k=2, wtype=wtype, seed=51)
    hl = em.make_host_layer(spec)
    x = (em.make_input(spec, T, seed=52) * np.float32(xstd)).astype(np.float32)
    print(f"range {em.TYPE_NAMES[wtype]} x~N(0,{xstd:g}) T={T}", flush=True)
    _check(hl, x)


@pytest.mark.parametrize("T", [1, 40, 600])
def test_bf16_weights_outside_fp16_range(gpu, T):
    spec = em.LayerSpec(d=512, d_ff=768, E=8, k=2, wtype=em.BF16, seed=53)
    hl = _layer(spec, [5e6, 5e-5])  # weights of ~1e5 and ~1e-6 by expert
    x = (em.make_input(spec, T, seed=54) * np.float32(1e3)).astype(np.float32)
    print(f"range bf16 weights 1e5 / 1e-6, x~N(0,1e3) T={T}", flush=True)
    _check(hl, x)


@pytest.mark.parametrize("T", [1, 200])
def test_bf16_shared_and_routed_split(gpu, T):
    """A DeepSeek-style BF16 layer with a shared expert: both run the split bf16 MFMA path at T = 200."""
    spec = em.LayerSpec(d=512, d_ff=384, E=16, k=4, wtype=em.BF16, bias_std=2.0, d_ff_shared=768, seed=55)
    hl = em.make_host_layer(spec)
    x = (em.make_input(spec, T, seed=56) * np.float32(30.0)).astype(np.float32)
    print(f"range bf16 shared T={T}", flush=True)
    _check(hl, x)
