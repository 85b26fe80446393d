"""The proven-picks router (moe_router_fast.hip, switched on by EMBER_ROUTER_FAST=1), taken by layer calls of
64 tokens and more whose router is a renormalised softmax (the reference's moe_ffn_f32_cpu with renorm,
utils.cpp:704-724, which reads only the picks' logits for the gates). Its int8 fast logits carry a bound
L <= l <= U on the reference's logit l, and only experts the bound cannot rule out get the exact FP64
chains.

  * check mode (EMBER_ROUTER_FAST_CHECK=1): every logit is computed exactly and held against its [L, U];
    one outside turns its token's picks to -1, so bit-exact routing here means every bound held;
  * normal mode: picks, gates and the whole dispatch equal the oracle's bit for bit, the logits are exact
    or a lower bound below every pick (router_logits_match), the output equals the exact router's
    (EMBER_ROUTER_FAST=0, the default) bit for bit, and most experts are ruled out (the fast path ran and
    pruned).

Inputs: seeded normals and rows built to stress the bound: magnitudes spread over 2^-60 .. 2^60, one
outlier per row, zero and sparse rows, duplicated router rows (exact ties), near-ties a few ulps apart,
rows whose logits overflow f32 (+-inf) and NaN inputs (those rows take exact logits throughout)."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import router_logits_match, same_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CASES = {
    # name: (spec kwargs, T)
    "qwen_e128_k8": (dict(d=2048, d_ff=256, E=128, k=8, wtype=em.Q8_0), 256),
    "mixtral_e8_k2": (dict(d=4096, d_ff=256, E=8, k=2, wtype=em.Q8_0), 96),
    "e200_k5_odd_d": (dict(d=96, d_ff=256, E=200, k=5, wtype=em.F32), 70),
    "e256_k16": (dict(d=512, d_ff=256, E=256, k=16, wtype=em.Q8_0), 130),
    "k_eq_e": (dict(d=256, d_ff=256, E=4, k=4, wtype=em.F32), 64),
}
KINDS = ["normal", "scaled", "outlier", "sparse", "ties", "near", "inf", "nan"]


def _inputs(spec, T, kind, seed):
    """A layer's host copy and T tokens for the given stress kind."""
    hl = em.make_host_layer(spec)
    E, d = spec.E, spec.d
    R = hl.router.reshape(E, d).copy()
    x = em.make_input(spec, T, seed=seed).astype(np.float32).copy()
    rng = np.random.default_rng(seed)
    if kind == "scaled":
        x *= np.exp2(rng.integers(-60, 61, size=(T, 1))).astype(np.float32)
        R *= np.exp2(rng.integers(-30, 31, size=(E, 1))).astype(np.float32)
    elif kind == "outlier":
        x[np.arange(T), rng.integers(0, d, size=T)] *= 1e4
        R[np.arange(E), rng.integers(0, d, size=E)] *= 1e3
    elif kind == "sparse":
        x[rng.random((T, d)) < 0.97] = 0.0
        x[0] = 0.0
        R[rng.random((E, d)) < 0.5] = 0.0
    elif kind == "ties":
        for e in range(1, E, 3):
            R[e] = R[0]
        x[1] = x[0]
    elif kind == "near":
        for e in range(1, min(E, 6)):
            R[e] = R[0]
            R[e, e % d] = np.nextafter(R[0, e % d], np.float32(np.inf))
    elif kind == "inf":
        s = np.sign(x[0]).astype(np.float32)
        R[E // 2] = 1e37 * s
        R[E // 2 + (1 if E > 1 else 0)] = -1e37 * s
    elif kind == "nan":
        x[3, 5] = np.nan
        x[T - 1, 0] = np.inf
    hl.router = np.ascontiguousarray(R.reshape(-1))
    return hl, x


def _call(dl, x, monkeypatch, **env):
    import torch

    for k_, v in env.items():
        monkeypatch.setenv(k_, v)
    T = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    scratch = torch.full((em.scratch_bytes(dl.desc, T),), 0xFF, dtype=torch.uint8, device="cuda")
    out, scratch = dl.forward(xd, scratch=scratch)
    torch.cuda.synchronize()
    for k_ in env:
        monkeypatch.delenv(k_)
    return out.cpu().numpy(), em.scratch_routing(dl.desc, T, scratch)


def _check_routing(hl, x, r, exact_logits):
    s = hl.spec
    lg = O.router_logits(x, hl.router)
    idx, gates = O.route(lg, s.k, renorm=True)
    if exact_logits:
        assert same_bits(r["logits"], lg), "logits"
    else:
        assert router_logits_match(r["logits"], lg, idx), "logits"
    assert np.array_equal(r["idx"], idx), np.argwhere(r["idx"] != idx)[:8]
    assert same_bits(r["gates"], gates), "gates"
    offsets, perm = O.dispatch(idx, s.E)
    assert np.array_equal(r["offsets"], offsets)
    assert np.array_equal(r["perm"][:offsets[-1]], perm[:offsets[-1]])
    return lg, idx


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("name", sorted(CASES))
def test_fast_router(gpu, monkeypatch, name, kind):
    kw, T = CASES[name]
    spec = em.LayerSpec(seed=11, **kw)
    hl, x = _inputs(spec, T, kind, seed=60 + KINDS.index(kind))
    dl = em.DeviceLayer.upload(hl)
    print(f"fast router {name} {kind} T={T}", flush=True)
    # check mode: every logit exact and inside its bounds
    _, rc = _call(dl, x, monkeypatch, EMBER_ROUTER_FAST="1", EMBER_ROUTER_FAST_CHECK="1")
    _check_routing(hl, x, rc, exact_logits=True)
    # normal mode against the exact router
    y, r = _call(dl, x, monkeypatch, EMBER_ROUTER_FAST="1")
    lg, idx = _check_routing(hl, x, r, exact_logits=False)
    y0, r0 = _call(dl, x, monkeypatch, EMBER_ROUTER_FAST="0")
    assert same_bits(r0["logits"], lg)
    assert same_bits(y, y0), "output differs from the exact router's"
    if kind in ("normal", "outlier") and spec.k < spec.E:
        # the bound rules most experts out: the fast path ran and pruned
        exact = (r["logits"].view(np.uint32) == lg.view(np.uint32)).sum(axis=1)
        print(f"  exact logits per token: mean {exact.mean():.2f} (k={spec.k}, E={spec.E})", flush=True)
        assert exact.mean() <= spec.k + max(2.0, 0.25 * (spec.E - spec.k)), exact.mean()
