"""Layers of two larger production MoE shapes, beyond BASELINE's configs, through every launch plan a
batch size selects (one-token fused launches, expert GEMVs, 64- and 256-token MFMA tiles, the shared
expert's side launches): a DeepSeek-V3-shaped layer (d 7168, 256 experts in 8 groups, top-8 sigmoid
router with selection bias and scale, shared expert; Q8_0) and a Qwen3-235B-shaped layer (d 4096, d_ff
1536, 128 experts, top-8 softmax; Q4_K with its prefill pack, and BF16). Each call: routing read back
bit-exact against the oracle (the reference's router, utils.cpp:704-836), the output within 2e-3 rel-L2
of the oracle's layer, and a second call with the same bits."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, router_logits_match, run_oracle, same_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SHAPES = {
    "deepseek_v3_q8": dict(d=7168, d_ff=2048, E=256, k=8, wtype=em.Q8_0, scoring=em.SCORE_SIGMOID, renorm=True,
                           bias_std=1.0, groups_n=8, groups_top=4, out_scale=2.5, d_ff_shared=2048),
    "qwen3_235b_q4k": dict(d=4096, d_ff=1536, E=128, k=8, wtype=em.Q4_K),
    "qwen3_235b_bf16": dict(d=4096, d_ff=1536, E=128, k=8, wtype=em.BF16),
}

_layers = {}


def _layer(name):
    import torch

    if name not in _layers:
        _layers.clear()
        spec = em.LayerSpec(seed=7, **SHAPES[name])
        hl = em.make_host_layer(spec)
        dl = em.DeviceLayer.upload(hl)
        pb = em.prefill_pack_bytes(dl.desc)
        if pb:
            buf = torch.empty(pb, dtype=torch.uint8, device="cuda")
            em.prefill_pack(dl.desc, buf)
            dl.tensors["pack"] = buf
        _layers[name] = (hl, dl)
    return _layers[name]


@pytest.mark.parametrize("T", [1, 4, 32, 256])
@pytest.mark.parametrize("name", sorted(SHAPES))
def test_model_shape_layer(gpu, name, T):
    import torch

    hl, dl = _layer(name)
    s = hl.spec
    x = em.make_input(s, T, seed=T)
    xd = torch.from_numpy(x).cuda()
    print(f"model shape {name} T={T} path={em.path(dl.desc, T)}", flush=True)
    out, scratch = dl.forward(xd)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    r = em.scratch_routing(dl.desc, T, scratch)
    lg = O.router_logits(x, hl.router)
    idx, gates = O.route(lg, s.k, renorm=s.renorm, sigmoid=s.scoring == em.SCORE_SIGMOID, bias=hl.bias,
                         groups_n=s.groups_n, groups_top=s.groups_top)
    assert np.array_equal(r["idx"], idx)
    assert same_bits(r["gates"], gates)
    assert router_logits_match(r["logits"], lg, idx)
    assert np.isfinite(y).all()
    err = rel_l2(y, run_oracle(hl, x))
    print(f"  rel-L2 {err:.2e}", flush=True)
    assert err < 2e-3, err
    y2, _ = dl.forward(xd)
    torch.cuda.synchronize()
    assert same_bits(y, y2.cpu().numpy()), "not deterministic"
