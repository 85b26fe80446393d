"""The 256-token-tile gate/up launch's tail split: when the work items (hit experts' m-tiles x d_ff / 128
column tiles) leave a partial last round on the CUs, the items of that round are split over K into up to 8
parts (each at least one K tile), whose raw gate / up dots a fixup launch sums in part order before the
SwiGLU epilogue. Held to the oracle (the reference's dequantize-then-F32 layer, utils.cpp:704-748) at the
2e-3 rel-L2 bar, to the unsplit launch (EMBER_TAIL_PARTS=1: only the f32 summation order of the tail tiles
differs, which can move the fp16 rounding of an h value by one ulp, 2^-11 relative, before the down
projection; 5e-4 rel-L2) and to itself (deterministic)."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, run_oracle, same_bits

pytestmark = pytest.mark.gpu


def _run(dl, x):
    import torch

    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    out, _ = dl.forward(xd)
    torch.cuda.synchronize()
    return out.cpu().numpy()


CASES = {
    # name: (spec kwargs, T); tiles: hit experts x d_ff / 128 against 256 CUs
    "q8_one_round_and_tail": (dict(d=512, d_ff=5120, E=8, k=2, wtype=em.Q8_0), 16),   # ~8 x 40 = 320
    "q8_partial_round": (dict(d=512, d_ff=1024, E=8, k=2, wtype=em.Q8_0), 8),         # <= 64 tiles
    "q4_partial_round": (dict(d=512, d_ff=1280, E=8, k=2, wtype=em.Q4_K), 12),        # <= 80 tiles
    "q8_short_k": (dict(d=128, d_ff=512, E=4, k=2, wtype=em.Q8_0), 8),                # 2 K tiles: 2 parts
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_tail_split(gpu, monkeypatch, name):
    import torch

    kw, T = CASES[name]
    spec = em.LayerSpec(seed=51, **kw)
    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    buf = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
    em.prefill_pack(dl.desc, buf)
    dl.tensors["pack"] = buf
    x = em.make_input(spec, T, seed=52)
    monkeypatch.setenv("EMBER_MOE_PATH", "gemm")  # the 256-token tiles
    monkeypatch.setenv("EMBER_TAIL_PARTS", "8")   # the split, also for these short K (by default K >= 64 tiles)
    assert em.path(dl.desc, T) & em.PATH_TILES256
    print(f"tail split {name} T={T}", flush=True)
    y = _run(dl, x)
    assert same_bits(y, _run(dl, x)), "not deterministic"
    monkeypatch.setenv("EMBER_TAIL_PARTS", "1")
    y_whole = _run(dl, x)
    err_whole = rel_l2(y, y_whole)
    err = rel_l2(y, run_oracle(hl, x))
    print(f"  vs unsplit {err_whole:.2e}, vs oracle {err:.2e}", flush=True)
    assert err_whole < 5e-4, err_whole
    assert err < 2e-3, err
