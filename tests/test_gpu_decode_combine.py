"""GPU tests of the one-token decode path (fused routing, expert GEMVs, the down launch with the combine
fused in): the output of a one-token call has the same bits as the same token's row of a two-token call
(the down launch then the combine launch: the per-token arithmetic does not depend on the batch), for
plain, scaled, DeepSeek-style (sigmoid, bias, groups), top-8 and shared-expert layers, over repeated
calls (the fused routing's flag words are re-armed every call)."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, run_oracle, same_bits

pytestmark = pytest.mark.gpu

CASES = {
    "mixtral_q8": dict(d=512, d_ff=1024, E=8, k=2, wtype=em.Q8_0),
    "qwen_q4k": dict(d=512, d_ff=768, E=16, k=4, wtype=em.Q4_K),
    "deepseek_bf16_shared": dict(d=256, d_ff=512, E=16, k=4, wtype=em.BF16, scoring=em.SCORE_SIGMOID, renorm=True,
                                 bias_std=1.0, groups_n=4, groups_top=2, out_scale=2.5, d_ff_shared=512),
    "f32": dict(d=256, d_ff=256, E=4, k=2, wtype=em.F32),
    # the fused down launch's limits: eight picks; six picks with a shared expert
    "qwen_top8_q4k": dict(d=512, d_ff=768, E=32, k=8, wtype=em.Q4_K),
    "top6_shared_bf16": dict(d=512, d_ff=384, E=32, k=6, wtype=em.BF16, scoring=em.SCORE_SIGMOID, renorm=True,
                             bias_std=2.0, d_ff_shared=768),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_one_token_matches_batch_row(gpu, monkeypatch, name):
    import torch

    spec = em.LayerSpec(**CASES[name], seed=31)
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    x2 = em.make_input(spec, 2)
    print(f"decode combine {name}", flush=True)
    assert em.path(dl.desc, 1) & em.PATH_DOWN1  # one token: the down launch with the combine fused in
    xd2 = torch.from_numpy(x2).cuda()
    # the two-token call on the expert GEMVs (the path one token takes; small layers with a shared expert
    # would pick the MFMA tiles at two tokens)
    monkeypatch.setenv("EMBER_MOE_PATH", "gemv")
    y2, _ = dl.forward(xd2)
    monkeypatch.delenv("EMBER_MOE_PATH")
    for rep in range(3):
        y1, _ = dl.forward(xd2[rep % 2:rep % 2 + 1].contiguous())
        torch.cuda.synchronize()
        assert same_bits(y1.cpu().numpy(), y2[rep % 2:rep % 2 + 1].cpu().numpy()), rep
    bar = 1e-4 if spec.wtype == em.F32 else 2e-3
    assert rel_l2(y1.cpu().numpy(), run_oracle(hl, x2[0:1])) < bar  # the last call's token: row 0
