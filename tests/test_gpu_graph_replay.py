"""Layer calls captured in a HIP graph (as an engine's decode-step graph holds them, model.cpp:1290-1321)
and replayed several times, with eager calls and synchronisations between the replays: every replay's output
must equal the eager call's bit for bit, on each launch plan — the one-token slice launch (per-call routing
tags, words cleared by the reduce launch), the one-token GEMV launches, and the 256-token tile launches of a
small batch (short tiles, the tail split and its fixup launch)."""
import numpy as np
import pytest

import ember_moe as em

pytestmark = pytest.mark.gpu

CASES = {
    # name: (spec kwargs, T, environment, the EMBER_PATH bits the call must take)
    "slices_q8": (dict(d=1024, d_ff=512, E=8, k=2, wtype=em.Q8_0), 1, {"EMBER_MOE_SLICES": "1"}, em.PATH_SLICES),
    "gemv_q4": (dict(d=1024, d_ff=512, E=8, k=2, wtype=em.Q4_K), 1, {"EMBER_MOE_SLICES": "0"}, em.PATH_GEMV),
    "tiles_tail_q8": (dict(d=512, d_ff=1024, E=8, k=2, wtype=em.Q8_0), 8, {"EMBER_MOE_PATH": "gemm",
                                                                           "EMBER_TAIL_PARTS": "8"}, em.PATH_TILES256),
    "tiles_q4_shared": (dict(d=512, d_ff=768, E=8, k=2, wtype=em.Q4_K, d_ff_shared=512), 24,
                        {"EMBER_MOE_PATH": "gemm"}, em.PATH_TILES256),
}
CALLS = 4  # layer calls per graph (two copies of the layer, alternating)


@pytest.mark.parametrize("name", sorted(CASES))
def test_graph_replays_match_eager(gpu, monkeypatch, name):
    import torch

    kw, T, env, bit = CASES[name]
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    spec = em.LayerSpec(seed=81, **kw)
    dl = em.DeviceLayer.upload(em.make_host_layer(spec))
    dl.tensors["pack"] = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
    em.prefill_pack(dl.desc, dl.tensors["pack"])
    dls = [dl, dl.clone()]
    assert em.path(dl.desc, T) & bit
    print(f"graph replay {name} T={T}", flush=True)
    x = torch.from_numpy(em.make_input(spec, T, seed=82)).cuda()
    out = torch.empty_like(x)
    scratch = torch.empty(em.scratch_bytes(dl.desc, T), dtype=torch.uint8, device="cuda")
    assert em.moe_ffn(dl.desc, x, T, out, scratch) == 0
    torch.cuda.synchronize()
    want = out.clone()

    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert em.moe_ffn(dl.desc, x, T, out, scratch) == 0  # warm on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        for i in range(CALLS):
            assert em.moe_ffn(dls[i % 2].desc, x, T, out, scratch) == 0
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), f"replay {rep}"
        # the program's own eager work between the replays, on the same scratch
        assert em.moe_ffn(dls[1].desc, x, T, out, scratch) == 0
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), want.view(torch.int32)), f"eager after replay {rep}"
