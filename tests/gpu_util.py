"""Helpers for the GPU parity tests: run the HIP path through the C ABI and the oracle on the
same seeded inputs, and compare them."""
import numpy as np

import ember_moe as em
from oracle import oracle as O


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def run_gpu(hl: em.HostLayer, x: np.ndarray, pack: bool = False):
    """Uploads the layer and x (pack: with the layer's prefill pack), runs ember_moe_ffn, returns out as
    numpy."""
    import torch

    dl = em.DeviceLayer.upload(hl)
    if pack:
        buf = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
        em.prefill_pack(dl.desc, buf)
        dl.tensors["pack"] = buf
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    out, _ = dl.forward(xd)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def run_oracle(hl: em.HostLayer, x: np.ndarray, nthreads: int = 0):
    s = hl.spec
    G, U, D = (hl.dequantized(n) for n in ("gate", "up", "down"))
    kw = {}
    if s.d_ff_shared:
        kw = dict(d_ff_sh=s.d_ff_shared, Gs=hl.dequantized("gate_sh"), Us=hl.dequantized("up_sh"),
                  Ds=hl.dequantized("down_sh"))
    return O.moe_layer(x, hl.router, G, U, D, s.d_ff, s.E, s.k, renorm=s.renorm,
                       sigmoid=s.scoring == em.SCORE_SIGMOID, bias=hl.bias, groups_n=s.groups_n,
                       groups_top=s.groups_top, scale=s.out_scale, Wsg=hl.shared_gate, nthreads=nthreads, **kw)


def same_bits(a, b) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(both_nan | (a.view(np.uint32) == b.view(np.uint32))))
