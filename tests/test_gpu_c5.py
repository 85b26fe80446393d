"""BASELINE config 5 at full size: the 32-layer random-init Mixtral-8x7B-architecture model with Q4_K
experts (ember_moe/mixtral.py), a 512-token seeded prompt through prefill, with the MoE FFN of several
layers checked against the CPU oracle inside the run:
  * routing of every prompt token of those layers (router logits, expert ids, gates) read back from the
    call's scratch, bit-exact against the oracle on the same inputs;
  * the FFN output of a seeded sample of tokens at the 2e-3 rel-L2 bar against the oracle's
    dequantize-then-F32 layer (the reference's path, utils.cpp:704-748);
then greedy decode steps: eager steps whose one-token MoE calls of the same layers (the decode branch,
model.cpp:757-762 / 1318-1321: the slice launch over the prefill pack) are checked the same way (routing
bit-exact, output at 2e-3 against the oracle on the decoded token's hidden state), and steps replayed from
the captured HIP graph, which must give the same tokens as the eager steps."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, router_logits_match, same_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu

LAYERS = (0, 13, 31)
SAMPLE = 4


def test_c5_per_layer_parity(gpu):
    import torch
    from ember_moe import mixtral

    spec = mixtral.MixtralSpec()
    T = 512
    model = mixtral.Mixtral(spec, max_ctx=T + 8, log=lambda *a: print(*a, flush=True))
    seen = {}

    def probe(l, h, f, scratch, L):
        if l in LAYERS and l not in seen:
            r = em.scratch_routing(L, h.shape[0], scratch)
            rows = np.sort(np.random.default_rng(l).choice(h.shape[0], SAMPLE, replace=False))
            seen[l] = (h.cpu().numpy(), f.cpu().numpy()[rows], rows, r)

    prompt = torch.from_numpy(np.random.default_rng(0).integers(0, spec.vocab, T)).cuda()
    model.probe = probe
    print("c5 prefill", flush=True)
    first = model.prefill(prompt)
    torch.cuda.synchronize()
    model.probe = None
    assert sorted(seen) == sorted(LAYERS)
    # decode: eager steps, with the one-token calls of the same layers captured at every step
    dec = {l: [] for l in LAYERS}

    def probe_dec(l, h, f, scratch, L):
        if l in LAYERS and h.shape[0] == 1:
            dec[l].append((h.cpu().numpy(), f.cpu().numpy(), em.scratch_routing(L, 1, scratch)))

    bits = em.path(model.layers[0], 1)
    assert bits & em.PATH_SLICES and bits & em.PATH_FUSED_ROUTE, bits
    model.probe = probe_dec
    print("c5 eager decode", flush=True)
    f_eager, toks_eager, _, _ = model.generate(prompt[:64], 4, use_graph=False)
    model.probe = None
    runs = [(int(f_eager[0]), toks_eager.cpu().numpy())]
    for l in LAYERS:
        h, f_rows, rows, r = seen[l]
        router = model.routers[l].cpu().numpy().reshape(-1)
        gate, up, down = (t.cpu().numpy() for t in model.experts[l])
        n_gu, n_dn = spec.E * spec.d_ff * spec.d, spec.E * spec.d * spec.d_ff
        G = em.dequantize(spec.expert_type, gate, n_gu)
        U = em.dequantize(spec.expert_type, up, n_gu)
        D = em.dequantize(spec.expert_type, down, n_dn)
        lg = O.router_logits(h, router)
        idx, gates = O.route(lg, spec.k)
        assert router_logits_match(r["logits"], lg, idx), l
        assert np.array_equal(r["idx"], idx) and same_bits(r["gates"], gates), l
        want = O.moe_layer(h[rows], router, G, U, D, spec.d_ff, spec.E, spec.k)
        err = rel_l2(f_rows, want)
        print(f"c5 layer {l}: routing of {T} tokens bit-exact, rel-L2 {err:.2e} over tokens {rows.tolist()}",
              flush=True)
        assert err < 2e-3
        assert len(dec[l]) == 4, len(dec[l])  # one call per decode step
        for step, (hd, fd, rd) in enumerate(dec[l]):
            lg = O.router_logits(hd, router)
            assert same_bits(rd["logits"], lg), (l, step)
            idx, gates = O.route(lg, spec.k)
            assert np.array_equal(rd["idx"], idx) and same_bits(rd["gates"], gates), (l, step)
            assert rd["conflict"] == 0
            err = rel_l2(fd, O.moe_layer(hd, router, G, U, D, spec.d_ff, spec.E, spec.k))
            print(f"c5 layer {l} decode step {step}: experts {idx[0].tolist()}, rel-L2 {err:.2e}", flush=True)
            assert err < 2e-3
        del G, U, D
    # graph replay of the decode steps gives the eager steps' tokens
    f0, toks, _, _ = model.generate(prompt[:64], 4, use_graph=True)
    runs.append((int(f0[0]), toks.cpu().numpy()))
    assert runs[0][0] == runs[1][0] and np.array_equal(runs[0][1], runs[1][1])
    assert int(first[0]) >= 0
