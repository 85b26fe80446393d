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


def router_logits_match(got, want, idx) -> bool:
    """The logits a layer call read back against the reference's (oracle) logits. Bit-equal, except where
    the proven-picks router (renormalised softmax routers, batches of EMBER_ROUTER_FAST_T tokens and more)
    ruled an expert out from its bounds: there it stores a lower bound of that expert's logit that lies
    strictly below every pick's logit. A row with a NaN logit (a non-finite input) is exact throughout."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    idx = np.asarray(idx)
    eq = (np.isnan(got) & np.isnan(want)) | (got.view(np.uint32) == want.view(np.uint32))
    for t in np.nonzero(~eq.all(axis=1))[0]:
        if np.isnan(want[t]).any():
            return False
        picks = idx[t][idx[t] >= 0]
        floor = want[t, picks].min()
        d = ~eq[t]
        if np.isin(np.nonzero(d)[0], picks).any():
            return False
        if not (np.all(got[t, d] < floor) and np.all(got[t, d] <= want[t, d])):
            return False
    return True
