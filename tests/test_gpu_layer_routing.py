"""Routing as ember_moe_ffn itself computes it, read back from the call's scratch
(ember_moe_scratch_routing) and compared bit for bit with the oracle.

At one token the router, the top-k, the gates and the dispatch run fused inside the gate/up expert
launch (every block recomputes them; block 0 writes them for the later launches); at 2..8 tokens a
small fused routing + dispatch kernel runs. Neither is the route_kernel that test_gpu_route.py checks
through ember_moe_route, so this test reads back logits, idx, gates, offsets, perm, pos, used and
n_used from layer calls and holds them to the reference's routing (utils.cpp:706-733 softmax, 758-820
DeepSeek router) and the stable-sort dispatch, including tied, NaN and +-inf logits.

The bounded wait of the fused routing is exercised from the host: with EMBER_MOE_TEST_ROUTE_NOPUBLISH=1
the router blocks do not publish their logits and every block must give up and compute the logits
itself; the layer's output must not change, and the fallback counter must say that it happened."""
import os

import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, router_logits_match, run_oracle, same_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _check_routing(hl, x, r):
    s = hl.spec
    T = x.shape[0]
    lg = O.router_logits(x, hl.router)
    idx, gates = O.route(lg, s.k, renorm=s.renorm, sigmoid=s.scoring == em.SCORE_SIGMOID, bias=hl.bias,
                         groups_n=s.groups_n, groups_top=s.groups_top)
    assert router_logits_match(r["logits"], lg, idx), "logits"
    assert np.array_equal(r["idx"], idx), (r["idx"], idx)
    assert same_bits(r["gates"], gates), (r["gates"], gates)
    offsets, perm = O.dispatch(idx, s.E)
    nslots = int(offsets[-1])
    assert np.array_equal(r["offsets"], offsets)
    assert np.array_equal(r["perm"][:nslots], perm[:nslots])
    # pos inverts perm over the picked slots; unpicked slots are -1
    want_pos = np.full(T * s.k, -1, np.int32)
    want_pos[perm[:nslots]] = np.arange(nslots, dtype=np.int32)
    assert np.array_equal(r["pos"], want_pos)
    used = np.flatnonzero(np.diff(offsets) > 0).astype(np.int32)
    assert r["n_used"] == used.size and np.array_equal(r["used"], used)
    # one token, softmax router: the pick set the expert launch proved from its fast logits equalled the
    # exact routing's (the scratch starts zeroed)
    assert r["mismatches"] == 0


def _run(dl, x):
    import torch

    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    T = x.shape[0]
    scratch = torch.zeros(em.scratch_bytes(dl.desc, T), dtype=torch.uint8, device="cuda")
    out, scratch = dl.forward(xd, scratch=scratch)
    torch.cuda.synchronize()
    return out.cpu().numpy(), em.scratch_routing(dl.desc, T, scratch)


SMALL = {
    "softmax-renorm": dict(d=256, d_ff=256, E=8, k=2, wtype=em.F32),
    "softmax-raw": dict(d=256, d_ff=256, E=8, k=2, wtype=em.F32, renorm=False),
    "wide-k8": dict(d=512, d_ff=256, E=128, k=8, wtype=em.Q8_0),
    "sigmoid-groups-bias": dict(d=512, d_ff=256, E=64, k=6, wtype=em.BF16, scoring=em.SCORE_SIGMOID, bias_std=2.0,
                                groups_n=8, groups_top=3),
    "softmax-bias-scale": dict(d=256, d_ff=256, E=16, k=4, wtype=em.F16, bias_std=1.0, out_scale=2.5),
}


@pytest.mark.parametrize("name", sorted(SMALL))
@pytest.mark.parametrize("T", range(1, 9))
def test_layer_routing_bit_exact(gpu, name, T):
    spec = em.LayerSpec(seed=3, **SMALL[name])
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    x = em.make_input(spec, T, seed=40 + T)
    print(f"layer routing {name} T={T}", flush=True)
    y, r = _run(dl, x)
    _check_routing(hl, x, r)
    bar = 1e-5 if spec.wtype == em.F32 else 2e-3
    assert rel_l2(y, run_oracle(hl, x)) < bar


def _edge_layer(T, kind):
    """A layer whose router makes tied, NaN or infinite logits for some tokens."""
    spec = em.LayerSpec(d=256, d_ff=256, E=16, k=4, wtype=em.F32, seed=5)
    hl = em.make_host_layer(spec)
    R = hl.router.reshape(spec.E, spec.d)
    x = em.make_input(spec, T, seed=77).copy()
    if kind == "ties":
        R[3] = R[1]       # experts 1, 3 and 9 always tie
        R[9] = R[1]
        R[12] = 0.0       # a zero logit
    elif kind == "inf":
        s = np.sign(x[0]).astype(np.float32)
        R[5] = 1e37 * s   # token 0: +inf for expert 5, -inf for expert 6
        R[6] = -1e37 * s
    elif kind == "nan":
        x[0, 7] = np.nan  # token 0: every logit NaN
    elif kind == "near":
        # logits closer than the fast logits' bound: expert 2 differs from expert 1 in one weight's last
        # bits, expert 4 by a relative 1e-6, expert 7 by 1e-3 (far enough to be proven apart)
        R[2] = R[1]
        R[2, 0] = np.nextafter(np.nextafter(R[1, 0], np.float32(np.inf)), np.float32(np.inf))
        R[4] = R[1] * np.float32(1 + 1e-6)
        R[7] = R[1] * np.float32(1 + 1e-3)
    hl.router = np.ascontiguousarray(R.reshape(-1))
    return hl, x


@pytest.mark.parametrize("kind", ["ties", "inf", "nan", "near"])
@pytest.mark.parametrize("T", [1, 2, 5, 8])
def test_layer_routing_edges(gpu, kind, T):
    hl, x = _edge_layer(T, kind)
    dl = em.DeviceLayer.upload(hl)
    print(f"layer routing edge {kind} T={T}", flush=True)
    y, r = _run(dl, x)
    _check_routing(hl, x, r)
    if kind in ("ties", "near"):
        assert rel_l2(y, run_oracle(hl, x)) < 1e-5


@pytest.mark.parametrize("seed", range(24))
def test_one_token_near_ties(gpu, seed):
    """One token whose k-th and (k+1)-th logits are nearly equal, at gaps from far below to far above
    what the fast logits can resolve: the exact routing decides wherever the proof cannot."""
    spec = em.LayerSpec(d=512, d_ff=256, E=8, k=2, wtype=em.F32, seed=200 + seed)
    hl = em.make_host_layer(spec)
    x = em.make_input(spec, 1, seed=300 + seed)
    R = hl.router.reshape(spec.E, spec.d)
    lg = O.router_logits(x, hl.router)[0]
    order = np.argsort(-lg, kind="stable")
    a, b = order[1], order[2]  # the second pick and the best unpicked expert
    gap = [0.0, 1e-9, 1e-7, 1e-5, 1e-4, 1e-3][seed % 6] * (1 if seed % 12 < 6 else -1)
    R[b] = R[a] * np.float32(1 + gap)  # expert b's logit ~ (1 + gap) times expert a's
    hl.router = np.ascontiguousarray(R.reshape(-1))
    dl = em.DeviceLayer.upload(hl)
    print(f"near tie seed={seed} gap={gap}", flush=True)
    y, r = _run(dl, x)
    _check_routing(hl, x, r)
    assert rel_l2(y, run_oracle(hl, x)) < 1e-5


FULL = {
    "c2": dict(d=4096, d_ff=14336, E=8, k=2, wtype=em.Q8_0),
    "c3": dict(d=2048, d_ff=768, E=128, k=8, wtype=em.Q4_K),
    "c4": dict(d=2048, d_ff=1408, E=64, k=6, wtype=em.BF16, bias_std=2.0, d_ff_shared=2816),
}


@pytest.mark.parametrize("name", sorted(FULL))
def test_layer_routing_full_size(gpu, name):
    spec = em.LayerSpec(seed=0, **FULL[name])
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    for T in (1, 2, 8):
        x = em.make_input(spec, T, seed=900 + T)
        print(f"layer routing full {name} T={T}", flush=True)
        _, r = _run(dl, x)
        _check_routing(hl, x, r)


def test_fused_routing_fallback(gpu, monkeypatch):
    """Router blocks that never publish: every block must compute the logits itself, with the same
    result, and the scratch's fallback counter must record it."""
    import torch

    spec = em.LayerSpec(d=1024, d_ff=512, E=8, k=2, wtype=em.Q8_0, seed=11)
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    x = em.make_input(spec, 1, seed=12)
    y0, r0 = _run(dl, x)
    assert r0["fallbacks"] == 0
    monkeypatch.setenv("EMBER_MOE_TEST_ROUTE_NOPUBLISH", "1")
    y1, r1 = _run(dl, x)
    monkeypatch.delenv("EMBER_MOE_TEST_ROUTE_NOPUBLISH")
    assert r1["fallbacks"] > 0, "the wait never gave up"
    assert same_bits(y1, y0)
    _check_routing(hl, x, r1)
    # and the next normal call is unaffected (the stale words were cleared)
    y2, r2 = _run(dl, x)
    assert r2["fallbacks"] == 0 and same_bits(y2, y0)



@pytest.mark.parametrize("E,k", [(8, 2), (16, 4)])
def test_fast_proof_conflict_poisons_output(gpu, monkeypatch, E, k):
    """A pick set proven from wrong fast logits must never yield plausible numbers. With
    EMBER_MOE_TEST_FAST_CORRUPT=1 the router blocks publish negated fast values under their tight bounds,
    so the other blocks prove the bottom k (the wrong experts) and stream them; block 0's exact routing
    (utils.cpp:708-733) contradicts the bounds. The call must then write NaN in every output row and set
    the per-call conflict word, while the routing record stays the exact one. (E, k) = (8, 2) takes the
    one-token down launch with the combine fused in, (16, 4) the down launch plus the combine. The scratch
    starts as 0xff bytes: the conflict word is reset by every call, not accumulated."""
    import torch

    spec = em.LayerSpec(d=1024, d_ff=512, E=E, k=k, wtype=em.Q8_0, seed=21)
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    x = em.make_input(spec, 1, seed=22)
    xd = torch.from_numpy(x).cuda()

    def run():
        scratch = torch.full((em.scratch_bytes(dl.desc, 1),), 0xFF, dtype=torch.uint8, device="cuda")
        out, scratch = dl.forward(xd, scratch=scratch)
        torch.cuda.synchronize()
        return out.cpu().numpy(), em.scratch_routing(dl.desc, 1, scratch)

    y0, r0 = run()
    assert r0["conflict"] == 0 and np.isfinite(y0).all()
    print(f"fast-proof conflict E={E} k={k}", flush=True)
    monkeypatch.setenv("EMBER_MOE_TEST_FAST_CORRUPT", "1")
    y1, r1 = run()
    monkeypatch.delenv("EMBER_MOE_TEST_FAST_CORRUPT")
    assert r1["conflict"] == 1, r1["conflict"]
    assert np.isnan(y1).all(), "a pick-set conflict produced finite output"
    assert r1["mismatches"] == (r0["mismatches"] + 1) % 2**64  # it grows from whatever the buffer held
    _check_exact_record(hl, x, r1)
    # the next call is clean again
    y2, r2 = run()
    assert r2["conflict"] == 0 and same_bits(y2, y0)


def _check_exact_record(hl, x, r):
    s = hl.spec
    lg = O.router_logits(x, hl.router)
    idx, gates = O.route(lg, s.k, renorm=s.renorm)
    assert router_logits_match(r["logits"], lg, idx)
    assert np.array_equal(r["idx"], idx) and same_bits(r["gates"], gates)
