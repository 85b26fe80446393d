"""Host data utilities (libember_moe_host.so): generator, fp16/bf16 encoders and the Q8_0 / Q4_K
quantizers. The product's host dequantizer must equal the oracle's (the reference's decoders)."""
import numpy as np

import ember_moe as em
from oracle import oracle as O


def test_normal_deterministic_and_sliceable():
    a = em.normal(100000, 3, 7)
    b = em.normal(100000, 3, 7)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, em.normal(100000, 4, 7))
    assert not np.array_equal(a, em.normal(100000, 3, 8))
    assert np.array_equal(a[:777], em.normal(777, 3, 7))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    c = em.normal(100000, 3, 7, 0.5, 0.02)
    assert abs(c.mean() - 0.5) < 1e-3 and abs(c.std() - 0.02) < 1e-3


def test_f16_encoder_matches_ieee_rne():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.standard_normal(20000) * 10 ** rng.uniform(-9, 5, 20000),
                        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 5.96e-8, 2.98e-8, 1e-10]]).astype(np.float32)
    want = v.astype(np.float16).view(np.uint16)
    got = np.array([em.host().ember_f32_to_f16(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, want)
    for h in range(0, 65536, 7):
        f = np.uint16(h).view(np.float16)
        if not np.isnan(f):
            assert em.host().ember_f16_to_f32(h) == np.float32(f)


def test_bf16_encoder_rne():
    import torch

    rng = np.random.default_rng(1)
    v = (rng.standard_normal(20000) * 10 ** rng.uniform(-20, 20, 20000)).astype(np.float32)
    want = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([em.host().ember_f32_to_bf16(float(x)) for x in v], np.uint16)
    assert np.array_equal(got, want)


def test_q8_0_quantizer_error_and_decode():
    x = em.normal(32 * 4096, 1, 1, 0.0, 0.02)
    raw = em.quantize(em.Q8_0, x)
    assert raw.size == 4096 * 34
    y = em.dequantize(em.Q8_0, raw, x.size)
    assert np.array_equal(y.view(np.uint32), O.dequant(em.Q8_0, raw, x.size).view(np.uint32))
    d = np.abs(x.reshape(-1, 32)).max(1) / 127
    # q is rounded against the unrounded scale, the decode uses its fp16 rounding: 0.5 step + 127 * 2^-11 step
    assert np.all(np.abs(x - y).reshape(-1, 32) <= d[:, None] * (0.5 + 127 * 2.0 ** -11) * (1 + 1e-3) + 1e-9)


def test_q4_k_quantizer_error_and_decode():
    x = em.normal(256 * 2048, 2, 1, 0.0, 0.02)
    raw = em.quantize(em.Q4_K, x)
    assert raw.size == 2048 * 144
    y = em.dequantize(em.Q4_K, raw, x.size)
    assert np.array_equal(y.view(np.uint32), O.dequant(em.Q4_K, raw, x.size).view(np.uint32))
    g = x.reshape(-1, 32)
    step = (g.max(1) - np.minimum(g.min(1), 0)) / 15
    err = np.abs(x - y).reshape(-1, 32).max(1)
    assert np.all(err <= step * 1.6 + 1e-6)  # within ~one quantization step of the group
    assert np.linalg.norm(x - y) / np.linalg.norm(x) < 0.12


def test_half_formats_roundtrip():
    x = em.normal(4096, 3, 1)
    for t in (em.F16, em.BF16, em.F32):
        raw = em.quantize(t, x)
        assert np.array_equal(em.dequantize(t, raw, x.size).view(np.uint32),
                              O.dequant(t, raw, x.size).view(np.uint32))
