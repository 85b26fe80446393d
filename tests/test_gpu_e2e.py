"""GPU test of the end-to-end harness (ember_moe/mixtral.py) on a tiny Mixtral-shaped model: the
decode steps replayed from the captured HIP graph produce the same greedy tokens as eager steps, and
the per-layer MoE FFN inside it is the C ABI call the layer tests check against the oracle."""
import numpy as np
import pytest

import ember_moe as em

pytestmark = pytest.mark.gpu


def test_graph_decode_matches_eager(gpu):
    import torch
    from ember_moe import mixtral

    spec = mixtral.MixtralSpec(n_layers=2, d=256, n_heads=4, n_kv=2, head_dim=64, E=4, k=2, d_ff=512,
                               vocab=1000, expert_type=em.Q4_K, expert_sets=2, seed=1)
    prompt = torch.from_numpy(np.random.default_rng(0).integers(0, spec.vocab, 24)).cuda()
    print("e2e tiny model", flush=True)
    runs = []
    for use_graph in (False, True):
        model = mixtral.Mixtral(spec, max_ctx=48, log=lambda *a: None)
        first, toks, _, _ = model.generate(prompt, 16, use_graph=use_graph)
        runs.append((int(first[0]), toks.cpu().numpy()))
    assert runs[0][0] == runs[1][0]
    assert np.array_equal(runs[0][1], runs[1][1])
    assert np.all((runs[1][1] >= 0) & (runs[1][1] < spec.vocab))
