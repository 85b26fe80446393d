"""GPU tests of the prefill pack (ember_moe_prefill_pack): the Q8_0 tile GEMMs reading packed tiles
give the same output bits as reading the ggml rows (same values, same arithmetic), on tile-aligned
and partial-tile shapes, with ragged expert segments, through the down projection's K split; Q4_K
stacks, whose pack feeds the same DMA tile kernels in place of the register-staged ones, give the same
bits as those wherever the down projection is not split over K (the factors and the order of the MFMA
accumulation are the same); and the oracle agrees at the quantized bar."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, run_oracle, same_bits

pytestmark = pytest.mark.gpu


def _run(hl, x, pack: bool):
    import torch

    dl = em.DeviceLayer.upload(hl)
    if pack:
        n = em.prefill_pack_bytes(dl.desc)
        assert n > 0
        buf = torch.empty(n, dtype=torch.uint8, device="cuda")
        em.prefill_pack(dl.desc, buf)
        dl.tensors["pack"] = buf
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    out, _ = dl.forward(xd)
    torch.cuda.synchronize()
    return out.cpu().numpy()


# more than 1.5 tokens per expert: the 256-token-tile GEMM (short segments skip their empty subtiles);
# d_ff 704 and d 576 leave partial n-tiles
@pytest.mark.parametrize("d,d_ff,E,k,T", [(512, 1024, 4, 2, 320), (576, 704, 4, 2, 300), (256, 512, 8, 2, 1024),
                                          (512, 1024, 4, 2, 64), (576, 704, 4, 2, 37), (256, 512, 8, 2, 150)])
def test_pack_same_bits_as_rows(gpu, d, d_ff, E, k, T):
    spec = em.LayerSpec(d=d, d_ff=d_ff, E=E, k=k, wtype=em.Q8_0, seed=21)
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, T)
    print(f"prefill pack d={d} d_ff={d_ff} E={E} T={T}", flush=True)
    y_rows = _run(hl, x, pack=False)
    y_pack = _run(hl, x, pack=True)
    assert same_bits(y_pack, y_rows)
    assert rel_l2(y_pack, run_oracle(hl, x)) < 2e-3


def test_pack_deepseek_style_with_shared_expert(gpu):
    """Sigmoid scoring, selection bias, groups, an output scale and a Q8_0 shared expert (its own GEMM,
    not in the pack): the routed experts read the pack, same bits."""
    spec = em.LayerSpec(d=512, d_ff=512, E=16, k=4, wtype=em.Q8_0, scoring=em.SCORE_SIGMOID, renorm=True,
                        bias_std=1.0, groups_n=4, groups_top=2, out_scale=2.5, d_ff_shared=1024, seed=29)
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, 400)
    print("prefill pack deepseek-style", flush=True)
    y_pack = _run(hl, x, pack=True)
    assert same_bits(y_pack, _run(hl, x, pack=False))
    assert rel_l2(y_pack, run_oracle(hl, x)) < 2e-3


# Q4_K: d, d_ff multiples of 256; more than 2 tokens per expert takes the 256-token tiles
@pytest.mark.parametrize("d,d_ff,E,k,T", [(512, 768, 8, 2, 320), (256, 512, 4, 2, 1000), (768, 512, 16, 4, 700),
                                          (512, 768, 8, 2, 40)])
def test_q4_k_pack_same_bits_as_register_staged(gpu, monkeypatch, d, d_ff, E, k, T):
    """Both runs forced onto the 256-token tiles (EMBER_MOE_PATH=gemm): the packed DMA kernel and the
    register-staged one form the same fp16 operands and pair the same K elements in each MFMA. (The DMA
    kernel's tail split, which sums the K parts of the last round's tiles separately, is off for the
    comparison: EMBER_TAIL_PARTS=1.)"""
    spec = em.LayerSpec(d=d, d_ff=d_ff, E=E, k=k, wtype=em.Q4_K, seed=24)
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, T)
    print(f"prefill pack q4_k d={d} d_ff={d_ff} E={E} T={T}", flush=True)
    y_default = _run(hl, x, pack=True)
    monkeypatch.setenv("EMBER_MOE_PATH", "gemm")
    monkeypatch.setenv("EMBER_TAIL_PARTS", "1")
    y_rows = _run(hl, x, pack=False)
    y_pack = _run(hl, x, pack=True)
    monkeypatch.delenv("EMBER_MOE_PATH")
    monkeypatch.delenv("EMBER_TAIL_PARTS")
    assert same_bits(y_pack, y_rows)
    assert rel_l2(y_default, run_oracle(hl, x)) < 2e-3


def test_q4_k_pack_with_k_split(gpu):
    """A long down projection (d_ff 4096) on few blocks: the DMA kernel splits its K and the combine adds
    the parts in a fixed order, so the bits differ from the unsplit kernel's but the oracle's bar holds."""
    spec = em.LayerSpec(d=256, d_ff=4096, E=4, k=2, wtype=em.Q4_K, seed=25)
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, 512)
    print("prefill pack q4_k K split", flush=True)
    y_pack = _run(hl, x, pack=True)
    assert rel_l2(y_pack, _run(hl, x, pack=False)) < 1e-5
    assert rel_l2(y_pack, run_oracle(hl, x)) < 2e-3


def test_pack_rejected_for_other_layers(gpu):
    import torch

    spec = em.LayerSpec(d=256, d_ff=512, E=4, k=2, wtype=em.F16, seed=2)
    dl = em.DeviceLayer.upload(em.make_host_layer(spec))
    assert em.prefill_pack_bytes(dl.desc) == 0
    buf = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(em.EmberError) as e:
        em.prefill_pack(dl.desc, buf)
    assert e.value.status == em.ERR_TYPE
    need = em.scratch_bytes(dl.desc, 4)
    dl.desc.prefill_pack = buf.data_ptr()  # a pack on a layer that has none: the call is refused
    assert em.scratch_bytes(dl.desc, 4) == 0
    x = torch.zeros(4, 256, device="cuda")
    out = torch.empty_like(x)
    scratch = torch.empty(need, dtype=torch.uint8, device="cuda")
    assert em.moe_ffn(dl.desc, x, 4, out, scratch) == em.ERR_TYPE


@pytest.mark.parametrize("wtype,d_ff,pack", [(em.Q8_0, 704, False), (em.Q8_0, 704, True), (em.Q4_K, 768, True)])
def test_64_token_tiles_forced(gpu, monkeypatch, wtype, d_ff, pack):
    """The 64-token-tile DMA kernel (a tuning choice, EMBER_MOE_PATH=skinny) agrees with the default
    kernel on the oracle's bar, with and without the pack (Q4_K: against its register-staged kernel)."""
    spec = em.LayerSpec(d=512, d_ff=d_ff, E=8, k=2, wtype=wtype, seed=23)
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, 90)
    print(f"64-token tiles forced, pack={pack}", flush=True)
    monkeypatch.setenv("EMBER_MOE_PATH", "skinny")
    y = _run(hl, x, pack=pack)
    if pack and wtype == em.Q8_0:
        assert same_bits(y, _run(hl, x, pack=False))  # packed tiles and the ggml rows: the same bits
    elif pack:  # the register-staged 64-token kernel pairs other K elements per MFMA: f32 rounding apart
        assert rel_l2(y, _run(hl, x, pack=False)) < 1e-5
    monkeypatch.delenv("EMBER_MOE_PATH")
    assert rel_l2(y, run_oracle(hl, x)) < 2e-3


# ---- BF16 layers: the pack holds row exponents, and the MFMA paths run fp16 operands (each weight row
# scaled by 2^-e, e putting its largest magnitude in [0.5, 1); the epilogue multiplies the column by 2^e)
# instead of the split bf16 MFMA (two products per weight)

def _bf16_scaled(spec, scales):
    """N(0, 0.02) stacks times a per-expert factor (cycled), as BF16."""
    s = spec
    hl = em.make_host_layer(s)

    def stack(name, rows, cols):
        v = em.normal(s.E * rows * cols, s.seed, 40 + len(name), 0.0, 0.02).reshape(s.E, rows, cols)
        v = v * np.array([scales[e % len(scales)] for e in range(s.E)], np.float32)[:, None, None]
        return em.quantize(em.BF16, np.ascontiguousarray(v, np.float32).reshape(-1))

    hl.gate = stack("gate", s.d_ff, s.d)
    hl.up = stack("up", s.d_ff, s.d)
    hl.down = stack("down_", s.d, s.d_ff)
    return hl


@pytest.mark.parametrize("T", [40, 600])
def test_bf16_pack_weights_outside_fp16_range(gpu, T):
    """Experts of ~1e5 and ~1e-6 weights (outside fp16's normal range) and x ~ N(0, 1e3): the row exponents
    keep the fp16 operands in range (T = 40: 64-token tiles, T = 600: 256-token tiles)."""
    spec = em.LayerSpec(d=512, d_ff=768, E=8, k=2, wtype=em.BF16, seed=53)
    hl = _bf16_scaled(spec, [5e6, 5e-5])
    x = (em.make_input(spec, T, seed=54) * np.float32(1e3)).astype(np.float32)
    print(f"bf16 pack range T={T}", flush=True)
    y = _run(hl, x, pack=True)
    want = run_oracle(hl, x)
    assert np.all(np.isfinite(y))
    assert rel_l2(y, want) < 2e-3


@pytest.mark.parametrize("T", [16, 200, 700])
def test_bf16_pack_with_shared_expert(gpu, T):
    """A DeepSeek-style BF16 layer (selection bias, shared expert, output scale): routed and shared experts
    take the fp16 path with the pack's exponents; the split path without the pack agrees at the bar."""
    spec = em.LayerSpec(d=512, d_ff=384, E=16, k=4, wtype=em.BF16, bias_std=2.0, d_ff_shared=768, out_scale=2.5,
                        seed=55)
    hl = em.make_host_layer(spec)
    # (x scaled by 10, not more: with larger logits the selection bias can pick four experts whose softmax
    # scores all underflow to 0, and the renormalisation then gives NaN gates, in the reference as here)
    x = (em.make_input(spec, T, seed=56) * np.float32(10.0)).astype(np.float32)
    print(f"bf16 pack shared T={T}", flush=True)
    y = _run(hl, x, pack=True)
    want = run_oracle(hl, x)
    assert np.all(np.isfinite(want)) and np.all(np.isfinite(y))
    assert rel_l2(y, want) < 2e-3
    assert rel_l2(_run(hl, x, pack=False), want) < 2e-3


def test_bf16_row_exponents(gpu):
    """The pack's exponents against numpy: frexp of each row's largest finite magnitude (0 for a row of
    zeros or of no finite value), clamped to [-120, 120]; rows holding Inf / NaN, huge, tiny and subnormal
    values included."""
    import torch

    spec = em.LayerSpec(d=256, d_ff=256, E=4, k=2, wtype=em.BF16, d_ff_shared=512, seed=57)
    hl = em.make_host_layer(spec)
    g = hl.gate.view(np.uint16).reshape(spec.E, spec.d_ff, spec.d).copy()
    bf = lambda v: (np.array([v], np.float32).view(np.uint32) >> 16).astype(np.uint16)[0]
    g[0, 0, :] = 0
    g[0, 1, 7] = bf(np.inf)
    g[0, 2, :] = bf(np.nan)
    g[0, 3, 5] = bf(-3e30)
    g[0, 4, :] = bf(1e-39)  # bf16 subnormal: frexp exponent -129, clamped
    g[0, 5, 9] = bf(-0.75)
    g[1, 6, :] = bf(np.float32(2.0 ** -100))
    hl.gate = g.reshape(-1).view(np.uint8).copy()
    dl = em.DeviceLayer.upload(hl)
    n = em.prefill_pack_bytes(dl.desc)
    buf = torch.zeros(n, dtype=torch.uint8, device="cuda")
    em.prefill_pack(dl.desc, buf)
    torch.cuda.synchronize()
    pack = buf.cpu().numpy()

    def want(u16, rows, cols):
        v = (u16.astype(np.uint32) << 16).view(np.float32).reshape(rows, cols).astype(np.float64)
        a = np.where(np.isfinite(v), np.abs(v), 0.0).max(axis=1)
        return np.clip(np.where(a > 0, np.frexp(a)[1], 0), -120, 120).astype(np.int16)

    al = lambda v: -(-v // 256) * 256
    E, d, f, fs = spec.E, spec.d, spec.d_ff, spec.d_ff_shared
    off = 0
    exps = {}
    # sections: gate, up, down, per-expert max of gate + up; the shared expert's the same
    for name, rows, cols, nexp in [("gate", E * f, d, E), ("up", E * f, d, E), ("down", E * d, f, E),
                                   ("gate_sh", fs, d, 1), ("up_sh", fs, d, 1), ("down_sh", d, fs, 1)]:
        got = pack[off:off + 2 * rows].view(np.int16)
        exps[name] = want(getattr(hl, name).view(np.uint16), rows, cols)
        assert np.array_equal(got, exps[name]), name
        off += al(2 * rows)
        if name.startswith("down"):
            g_, u_ = exps["gate" + name[4:]], exps["up" + name[4:]]
            hmax = (g_.astype(np.int32) + u_).reshape(nexp, -1).max(axis=1)
            assert np.array_equal(pack[off:off + 2 * nexp].view(np.int16), hmax), name + " max"
            off += al(2 * nexp)
    assert off == n
