"""The 256-token DMA tile kernels' short variant: a launch of at most 64 tokens has no segment, hence no tile,
of more than 64 rows (a token picks an expert once), so its LDS stages hold 64 activation rows and five
stages fit (four tiles in flight instead of two). It multiplies the same fragments in the same order as the
three-stage kernel, so its outputs are bit-identical to it (EMBER_GEMM_SHORT=0 forces the three-stage
kernel), and held to the oracle (utils.cpp:704-748) at the 2e-3 rel-L2 bar; 65 tokens take the three-stage
kernel."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, run_oracle, same_bits

pytestmark = pytest.mark.gpu


def _run(dl, x):
    import torch

    out, _ = dl.forward(torch.from_numpy(np.ascontiguousarray(x)).cuda())
    torch.cuda.synchronize()
    return out.cpu().numpy()


CASES = {
    # name: (spec kwargs, T, prefill pack)
    "q8_pack": (dict(d=512, d_ff=1024, E=8, k=2, wtype=em.Q8_0), 24, True),
    "q8_rows": (dict(d=512, d_ff=1024, E=8, k=2, wtype=em.Q8_0), 24, False),
    "q4_pack_64": (dict(d=512, d_ff=768, E=4, k=2, wtype=em.Q4_K), 64, True),  # 64 tokens: the limit
    "q4_pack_65": (dict(d=512, d_ff=768, E=4, k=2, wtype=em.Q4_K), 65, True),  # past it
    "q8_shared": (dict(d=512, d_ff=512, E=8, k=2, wtype=em.Q8_0, d_ff_shared=1024), 40, True),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_short_tiles_same_bits(gpu, monkeypatch, name):
    import torch

    kw, T, pack = CASES[name]
    spec = em.LayerSpec(seed=61, **kw)
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    if pack:
        buf = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
        em.prefill_pack(dl.desc, buf)
        dl.tensors["pack"] = buf
    x = em.make_input(spec, T, seed=62)
    monkeypatch.setenv("EMBER_MOE_PATH", "gemm")  # the 256-token tiles
    monkeypatch.setenv("EMBER_MOE_SHARED_PATH", "gemm")
    monkeypatch.setenv("EMBER_TAIL_PARTS", "1")  # (the tail split is the same in both; off keeps it simple)
    assert em.path(dl.desc, T) & em.PATH_TILES256
    print(f"short tiles {name} T={T}", flush=True)
    y = _run(dl, x)
    monkeypatch.setenv("EMBER_GEMM_SHORT", "0")
    y3 = _run(dl, x)
    assert same_bits(y, y3)
    err = rel_l2(y, run_oracle(hl, x))
    print(f"  rel-L2 vs oracle {err:.2e}", flush=True)
    assert err < 2e-3, err
