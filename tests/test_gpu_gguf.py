"""GPU tests of quantized residency: a layer read from a GGUF file and uploaded in its encoding by
ember_gguf_upload_layer runs through ember_moe_ffn to the same output bits as the same bytes
uploaded directly, and to the oracle at the format's bar."""
import numpy as np
import pytest

import ember_moe as em
from ember_moe import gguf_writer as gw
from gpu_util import rel_l2, run_gpu, run_oracle, same_bits

pytestmark = pytest.mark.gpu


def _run_from_gguf(path, layer, x):
    import torch

    with em.Gguf(path) as g:
        m = g.moe_layer(layer)
        need = em.gguf_layer_bytes(m)
        dev = torch.empty(need, dtype=torch.uint8, device="cuda")
        L = em.gguf_upload_layer(m, dev)
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    out = torch.empty_like(xd)
    scratch = torch.empty(em.scratch_bytes(L, x.shape[0]), dtype=torch.uint8, device="cuda")
    st = em.moe_ffn(L, xd, x.shape[0], out, scratch)
    assert st == em.OK, em.strerror(st)
    torch.cuda.synchronize()
    return out.cpu().numpy(), L


@pytest.mark.parametrize("wtype,T", [(em.Q8_0, 1), (em.Q8_0, 40), (em.Q4_K, 5)])
def test_mixtral_layer_from_gguf(gpu, tmp_path, wtype, T):
    spec = em.LayerSpec(d=512, d_ff=768, E=8, k=2, wtype=wtype, seed=11)
    hl = em.make_host_layer(spec)
    other = em.make_host_layer(em.LayerSpec(**{**spec.__dict__, "seed": 12}))
    p = str(tmp_path / "mixtral.gguf")
    gw.write_gguf(p, gw.moe_meta("llama", hl, 2), gw.moe_layer_tensors(other, 0) + gw.moe_layer_tensors(hl, 1))
    x = em.make_input(spec, T)
    print(f"gguf llama {em.TYPE_NAMES[wtype]} T={T}", flush=True)
    y, L = _run_from_gguf(p, 1, x)
    assert (L.renorm, L.gate_type, L.E, L.k) == (1, wtype, 8, 2)
    assert same_bits(y, run_gpu(hl, x))  # the same bytes on the device: the same kernels, the same bits
    assert rel_l2(y, run_oracle(hl, x)) < 2e-3


def test_deepseek_layer_from_gguf_with_bf16_router(gpu, tmp_path):
    spec = em.LayerSpec(d=256, d_ff=512, E=16, k=4, wtype=em.Q8_0, scoring=em.SCORE_SIGMOID, renorm=True,
                        bias_std=1.0, groups_n=4, groups_top=2, out_scale=2.5, d_ff_shared=512, seed=5)
    hl = em.make_host_layer(spec)
    p = str(tmp_path / "ds.gguf")
    gw.write_gguf(p, gw.moe_meta("deepseek2", hl, 1), gw.moe_layer_tensors(hl, 0, router_type=em.BF16))
    x = em.make_input(spec, 6)
    print("gguf deepseek2 T=6", flush=True)
    y, L = _run_from_gguf(p, 0, x)
    assert (L.scoring, L.groups_n, L.groups_top, L.d_ff_shared) == (em.SCORE_SIGMOID, 4, 2, 512)
    # the file's router is bf16: the device holds it widened to f32, exactly
    hl_bf = em.HostLayer(**{**hl.__dict__, "router": em.dequantize(em.BF16, em.quantize(em.BF16, hl.router), spec.E * spec.d)})
    assert same_bits(y, run_gpu(hl_bf, x))
    assert rel_l2(y, run_oracle(hl_bf, x)) < 2e-3


def test_upload_rejects_small_buffer_and_unsupported_type(gpu, tmp_path):
    import torch

    spec = em.LayerSpec(d=256, d_ff=512, E=4, k=2, wtype=em.Q8_0, seed=1)
    hl = em.make_host_layer(spec)
    t = gw.moe_layer_tensors(hl, 0)
    p = str(tmp_path / "a.gguf")
    gw.write_gguf(p, gw.moe_meta("llama", hl, 1), t)
    with em.Gguf(p) as g:
        m = g.moe_layer(0)
        dev = torch.empty(em.gguf_layer_bytes(m) - 256, dtype=torch.uint8, device="cuda")
        with pytest.raises(em.EmberError) as e:
            em.gguf_upload_layer(m, dev)
        assert e.value.status == em.ERR_SCRATCH
    # Q4_0 experts (type 2): read fine, but not an encoding the FFN runs
    q40 = [(n, 2 if "exps" in n else ty, ne, np.zeros(em.host().ember_ggml_nbytes(2, int(np.prod(ne))), np.uint8)
            if "exps" in n else raw) for n, ty, ne, raw in t]
    p2 = str(tmp_path / "q40.gguf")
    gw.write_gguf(p2, gw.moe_meta("llama", hl, 1), q40)
    with em.Gguf(p2) as g:
        m = g.moe_layer(0)
        dev = torch.empty(em.gguf_layer_bytes(m), dtype=torch.uint8, device="cuda")
        with pytest.raises(em.EmberError) as e:
            em.gguf_upload_layer(m, dev)
        assert e.value.status == em.ERR_TYPE


@pytest.mark.parametrize("T", [1, 12])
def test_qwen2moe_gated_shared_from_gguf(gpu, tmp_path, T):
    spec = em.LayerSpec(d=512, d_ff=256, E=16, k=4, wtype=em.Q8_0, renorm=False, d_ff_shared=512, shared_gated=True,
                        seed=8)
    hl = em.make_host_layer(spec)
    p = str(tmp_path / "q2.gguf")
    gw.write_gguf(p, gw.moe_meta("qwen2moe", hl, 1), gw.moe_layer_tensors(hl, 0))
    x = em.make_input(spec, T)
    print(f"gguf qwen2moe gated shared T={T}", flush=True)
    y, L = _run_from_gguf(p, 0, x)
    assert (L.renorm, L.d_ff_shared) == (0, 512) and L.shared_gate
    assert same_bits(y, run_gpu(hl, x))
    assert rel_l2(y, run_oracle(hl, x)) < 2e-3
