"""GPU parity at the BASELINE configs' full layer sizes.

Tokens are independent in the reference (one moe_ffn_f32_cpu call per token), so at sizes where the
oracle cannot finish every token in seconds it checks a seeded sample of tokens of the same batch:
the sample's rows of the GPU output must match the oracle run on the sample alone. Routing (logits,
experts, gates) is checked bit-exact on every token. The largest batches (a 16384-token Mixtral-shaped
prefill, 32768 tokens at the Qwen shape: 262144 routed rows) exercise the multi-block dispatch and every
index of the scratch at sizes eight times the BASELINE configs'."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, router_logits_match, same_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CONFIGS = {
    "c2": dict(d=4096, d_ff=14336, E=8, k=2, wtype=em.Q8_0),
    "c3": dict(d=2048, d_ff=768, E=128, k=8, wtype=em.Q4_K),
    "c4": dict(d=2048, d_ff=1408, E=64, k=6, wtype=em.BF16, bias_std=2.0, d_ff_shared=2816),
}
_layers = {}


def _layer(name):
    if name not in _layers:
        spec = em.LayerSpec(seed=0, **CONFIGS[name])
        hl = em.make_host_layer(spec)
        f32 = {n: hl.dequantized(n) for n in ("gate", "up", "down")}
        if spec.d_ff_shared:
            f32.update({n: hl.dequantized(n) for n in ("gate_sh", "up_sh", "down_sh")})
        _layers.clear()  # keep one full layer resident on the host at a time
        _layers[name] = (hl, em.DeviceLayer.upload(hl), f32)
    return _layers[name]


@pytest.mark.parametrize("name,T,sample", [("c2", 1, 1), ("c2", 8, 8), ("c2", 128, 12), ("c2", 2048, 12),
                                           ("c3", 1, 1), ("c3", 32, 32), ("c3", 4096, 24),
                                           ("c4", 1, 1), ("c4", 2048, 24),
                                           # long prefills: 32768 and 262144 dispatch slots
                                           ("c2", 16384, 8), ("c3", 32768, 16)])
def test_full_size_layer(gpu, name, T, sample):
    import torch

    hl, dl, f32 = _layer(name)
    s = hl.spec
    x = em.make_input(s, T, seed=1000 + T)
    print(f"full-size {name} T={T}", flush=True)
    xd = torch.from_numpy(x).cuda()
    out, scratch = dl.forward(xd)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    assert np.all(np.isfinite(y))
    # routing on every token, as this call computed it
    r = em.scratch_routing(dl.desc, T, scratch)
    lg = O.router_logits(x, hl.router)
    idx, gates = O.route(lg, s.k, renorm=s.renorm, bias=hl.bias)
    assert router_logits_match(r["logits"], lg, idx)
    assert np.array_equal(r["idx"], idx) and same_bits(r["gates"], gates)
    offsets, perm = O.dispatch(idx, s.E)
    assert np.array_equal(r["offsets"], offsets) and np.array_equal(r["perm"], perm)
    rows = np.sort(np.random.default_rng(T).choice(T, size=min(sample, T), replace=False))
    kw = {}
    if s.d_ff_shared:
        kw = dict(d_ff_sh=s.d_ff_shared, Gs=f32["gate_sh"], Us=f32["up_sh"], Ds=f32["down_sh"])
    want = O.moe_layer(x[rows], hl.router, f32["gate"], f32["up"], f32["down"], s.d_ff, s.E, s.k, renorm=s.renorm,
                       bias=hl.bias, **kw)
    err = rel_l2(y[rows], want)
    print(f"  rel-L2 {err:.2e} over {len(rows)} tokens")
    assert err < 2e-3
