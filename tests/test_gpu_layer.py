"""GPU parity of the whole MoE FFN layer through the C ABI, against the oracle.

Bars (north_star): F32 experts max-abs 1e-4 and rel-L2 1e-5 against the reference's CPU result;
BF16 / F16 / Q8_0 / Q4_K rel-L2 2e-3 against the reference's dequantize-then-F32 result."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, run_gpu, run_oracle
from golden_util import f32, load_cases

pytestmark = pytest.mark.gpu

F32_MAXABS, F32_RELL2, Q_RELL2 = 1e-4, 1e-5, 2e-3


def check(spec, T, seed=None, pack=False):
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, T, seed)
    print(f"layer {em.TYPE_NAMES[spec.wtype]} d={spec.d} d_ff={spec.d_ff} E={spec.E} k={spec.k} T={T} pack={pack}",
          flush=True)
    y = run_gpu(hl, x, pack=pack)
    want = run_oracle(hl, x)
    assert np.all(np.isfinite(y))
    if spec.wtype == em.F32 and (spec.d_ff_shared == 0 or spec.shared_type in (None, em.F32)):
        assert np.max(np.abs(y - want)) < F32_MAXABS
        assert rel_l2(y, want) < F32_RELL2
    else:
        assert rel_l2(y, want) < Q_RELL2
    return y, want


def test_c1_golden(gpu):
    """BASELINE config 1 against the reference's own output bits (tests/golden/c1_layer.npz)."""
    spec = em.LayerSpec(d=256, d_ff=688, E=8, k=2, wtype=em.F32, seed=0)
    hl = em.make_host_layer(spec)
    for name, c in load_cases("c1_layer.npz").items():
        s = em.LayerSpec(**{**spec.__dict__, "renorm": bool(c["renorm"])})
        hl.spec = s
        x = em.make_input(s, int(c["T"]))
        print("c1", name, flush=True)
        y = run_gpu(hl, x)
        want = f32(c["out_bits"])
        assert np.max(np.abs(y - want)) < F32_MAXABS, name
        assert rel_l2(y, want) < F32_RELL2, name


@pytest.mark.parametrize("T", [1, 2, 5, 16, 17, 40, 64])
@pytest.mark.parametrize("renorm", [True, False])
def test_f32_small(gpu, T, renorm):
    check(em.LayerSpec(d=96, d_ff=160, E=8, k=2, wtype=em.F32, renorm=renorm, seed=3, weight_std=0.3,
                       router_std=0.3), T)


@pytest.mark.parametrize("wtype", [em.Q8_0, em.BF16, em.F16])
@pytest.mark.parametrize("T", [1, 3, 8, 33])
def test_q8_bf16_f16(gpu, wtype, T):
    check(em.LayerSpec(d=512, d_ff=384, E=8, k=2, wtype=wtype, seed=5), T)


@pytest.mark.parametrize("T", [1, 4, 32, 70])
def test_q4_k(gpu, T):
    check(em.LayerSpec(d=512, d_ff=768, E=16, k=4, wtype=em.Q4_K, seed=6), T)


@pytest.mark.parametrize("T", [1, 9])
def test_deepseek_shared_bias_scale(gpu, T):
    """C4-style router: softmax with a seeded selection bias ~ N(0, 2), a shared expert, a scale."""
    check(em.LayerSpec(d=256, d_ff=192, E=16, k=6, wtype=em.BF16, bias_std=2.0, d_ff_shared=384, out_scale=2.5,
                       seed=7), T)


@pytest.mark.parametrize("wtype,T", [(em.Q8_0, 64), (em.Q8_0, 300), (em.Q4_K, 200), (em.BF16, 130), (em.F16, 96)])
def test_grouped_gemm_path(gpu, wtype, T):
    """A few dozen tokens per expert: the 64-token-tile MFMA GEMM (Q8_0: the 256-token-tile kernel,
    which it takes from 1.5 tokens per expert on); skewed routing (E 32, top-8) leaves ragged tiles."""
    check(em.LayerSpec(d=512, d_ff=768, E=32, k=8, wtype=wtype, seed=11), T)


@pytest.mark.parametrize("wtype,T", [(em.Q8_0, 512), (em.Q4_K, 700), (em.BF16, 450), (em.F16, 520)])
def test_large_tile_gemm_path(gpu, wtype, T):
    """More than ~96 tokens per expert: the 256-token-tile MFMA GEMM (ragged last tiles)."""
    check(em.LayerSpec(d=512, d_ff=768, E=8, k=2, wtype=wtype, seed=12), T)


@pytest.mark.parametrize("T", [64, 257, 600])
def test_grouped_gemm_shared_bias(gpu, T):
    check(em.LayerSpec(d=256, d_ff=192, E=16, k=6, wtype=em.BF16, bias_std=2.0, d_ff_shared=384, out_scale=2.5,
                       seed=7), T)


@pytest.mark.parametrize("T", [1, 6])
def test_sigmoid_groups(gpu, T):
    check(em.LayerSpec(d=128, d_ff=256, E=32, k=4, wtype=em.Q8_0, scoring=em.SCORE_SIGMOID, bias_std=0.5, groups_n=8,
                       groups_top=3, seed=8), T)


def test_k_greater_than_e(gpu):
    check(em.LayerSpec(d=64, d_ff=128, E=4, k=6, wtype=em.F32, seed=9), 5)


def test_deterministic(gpu):
    spec = em.LayerSpec(d=512, d_ff=768, E=16, k=4, wtype=em.Q4_K, seed=6)
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, 40)
    a = run_gpu(hl, x)
    b = run_gpu(hl, x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_t_zero_and_errors(gpu):
    import torch

    spec = em.LayerSpec(d=256, d_ff=256, E=8, k=2, wtype=em.Q8_0, seed=1)
    dl = em.DeviceLayer.upload(em.make_host_layer(spec))
    x = torch.zeros((4, 256), device="cuda")
    out = torch.full((4, 256), 7.0, device="cuda")
    need = em.scratch_bytes(dl.desc, 4)
    scratch = torch.empty(need, dtype=torch.uint8, device="cuda")
    assert em.moe_ffn(dl.desc, x, 0, out, scratch) == em.OK
    assert em.moe_ffn(dl.desc, x, 4, out, scratch, scratch_nbytes=need - 1) == em.ERR_SCRATCH
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)  # nothing ran
    assert em.moe_ffn(dl.desc, x, 4, out, scratch) == em.OK
    torch.cuda.synchronize()
    assert not torch.all(out == 7.0)


@pytest.mark.parametrize("forced", ["gemv", None])
@pytest.mark.parametrize("T", [2, 4, 6])
@pytest.mark.parametrize("shape", ["c4-like", "mixtral-like-f16", "mixed-types"])
def test_shared_expert_multi_token_gemv(gpu, monkeypatch, shape, T, forced):
    """A shared expert riding in the multi-token decode launches (one more segment of the routed GEMV
    launches when its types match the routed experts'; its own launches when they differ). EMBER_MOE_PATH
    =gemv forces the GEMV for the routed experts; unforced, each layer takes its own path choice."""
    if forced:
        monkeypatch.setenv("EMBER_MOE_PATH", forced)
    if shape == "c4-like":
        spec = em.LayerSpec(d=2048, d_ff=1408, E=64, k=6, wtype=em.BF16, bias_std=2.0, d_ff_shared=2816, seed=21)
    elif shape == "mixtral-like-f16":
        spec = em.LayerSpec(d=1024, d_ff=3584, E=8, k=2, wtype=em.F16, d_ff_shared=1024, out_scale=1.5, seed=22)
    else:  # BF16 routed experts with a Q8_0 shared expert
        spec = em.LayerSpec(d=1024, d_ff=768, E=16, k=4, wtype=em.BF16, d_ff_shared=1536, shared_type=em.Q8_0,
                            seed=23)
    check(spec, T, seed=300 + T)


@pytest.mark.parametrize("T", [16, 100, 300])
@pytest.mark.parametrize("wtype,shared_type,pack,gated", [(em.BF16, None, True, False), (em.BF16, None, False, False),
                                                          (em.Q8_0, em.BF16, True, False), (em.F16, None, False, False),
                                                          (em.Q8_0, None, False, True)])
def test_shared_expert_k_split(gpu, wtype, shared_type, pack, gated, T):
    """The shared expert's dense launches on 64-token tiles split over K when they have few blocks (at this
    shape 8 parts at T = 16, 2 at T = 100, none at T = 300): raw partial gate / up dots finished by a SwiGLU
    pass, down partials summed by the combine in part order; BF16 with the pack (fp16) and without (split
    bf16), a Q8_0 shared expert (its DMA kernel splits only down), qwen2moe's gated shared expert."""
    check(em.LayerSpec(d=1024, d_ff=512, E=16, k=4, wtype=wtype, d_ff_shared=1024, shared_type=shared_type,
                       shared_gated=gated, renorm=not gated, seed=61), T, pack=pack)


@pytest.mark.parametrize("wtype,T", [(em.BF16, 1), (em.BF16, 3), (em.BF16, 40), (em.BF16, 300), (em.Q8_0, 1),
                                     (em.Q8_0, 70), (em.F32, 5)])
def test_qwen2moe_gated_shared_expert(gpu, wtype, T):
    """qwen2moe (graph_ir.cpp:694-705): raw gates; the shared expert's row scaled by
    sigmoid(ffn_gate_inp_shexp . x) per token, then added. One token: the shared expert rides in the
    routed decode launches; many: its own MFMA launches."""
    check(em.LayerSpec(d=512, d_ff=256, E=16, k=4, wtype=wtype, renorm=False, d_ff_shared=1024, shared_gated=True,
                       seed=41), T)


def test_device_layer_clone(gpu):
    """DeviceLayer.clone (the bench's copies of a layer, prefill pack included): the same output bits at
    other addresses."""
    import torch

    spec = em.LayerSpec(d=512, d_ff=512, E=8, k=2, wtype=em.Q8_0, seed=71)
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    dl.tensors["pack"] = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
    em.prefill_pack(dl.desc, dl.tensors["pack"])
    c = dl.clone()
    assert c.desc.gate != dl.desc.gate and c.desc.prefill_pack not in (0, dl.desc.prefill_pack)
    for T in (1, 8, 300):
        x = torch.from_numpy(em.make_input(spec, T, seed=72)).cuda()
        y0, _ = dl.forward(x)
        y1, _ = c.forward(x)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int32), y1.view(torch.int32)), T
