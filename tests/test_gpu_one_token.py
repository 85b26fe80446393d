"""The one-token (decode, T = 1) paths of ember_moe_ffn, each checked through the C ABI:

  SLICES  (with a Q8_0 / Q4_K prefill pack, by default when the slices give every CU a block) the whole
          layer in one launch over 64-column slices of d_ff (each block: its slice's gate/up rows, SwiGLU,
          the matching down columns streamed from the pack's tiles) plus an ordered reduce of the slices'
          partial outputs;
  GEMV    (EMBER_MOE_SLICES=0, or no pack) the fused gate/up GEMV, then the down launch (with the combine
          fused in for top-1/2 layers).

Each is held to the oracle (the reference's dequantize-then-F32 layer, utils.cpp:704-748 for the softmax
router, 758-836 for the DeepSeek-style one) at the 2e-3 rel-L2 bar with the routing read back bit-exact.
SLICES differs from GEMV only in the f32 summation order for Q8_0 and, for Q4_K, in the pack's fp16 group
factors. Also: determinism, a pick set proven from corrupted fast logits (NaN rows and the per-call
conflict word), and the Mixtral-shaped calls of configs 2 (Q8_0) and 5 (Q4_K) that config 5's decode
tokens/s rests on (model.cpp:757-762 on the CPU, 1318-1321 in the CUDA decode graph)."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import rel_l2, run_oracle, same_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu

PATHS = {  # name: (environment, the EMBER_PATH bit it must select)
    # (EMBER_MOE_SLICES=1: also layers with fewer slices than CUs, which by default take the GEMV path)
    "slices": ({"EMBER_MOE_SLICES": "1"}, em.PATH_SLICES),
    "gemv": ({"EMBER_MOE_SLICES": "0"}, em.PATH_GEMV),
}


def _device_layer(spec, pack=True):
    import torch

    hl = em.make_host_layer(spec)
    dl = em.DeviceLayer.upload(hl)
    if pack:
        buf = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
        em.prefill_pack(dl.desc, buf)
        dl.tensors["pack"] = buf
    return hl, dl


def _run(dl, x):
    import torch

    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    scratch = torch.full((em.scratch_bytes(dl.desc, x.shape[0]),), 0xFF, dtype=torch.uint8, device="cuda")
    out, scratch = dl.forward(xd, scratch=scratch)
    torch.cuda.synchronize()
    return out.cpu().numpy(), em.scratch_routing(dl.desc, x.shape[0], scratch)


def _on_path(monkeypatch, dl, name):
    env, bit = PATHS[name]
    monkeypatch.delenv("EMBER_MOE_SLICES", raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    bits = em.path(dl.desc, 1)
    assert bits & bit and bits & em.PATH_FUSED_ROUTE, (name, bits)
    if name == "gemv":
        assert not bits & em.PATH_SLICES


def _check_routing(hl, x, r):
    s = hl.spec
    lg = O.router_logits(x, hl.router)
    assert same_bits(r["logits"], lg)
    idx, gates = O.route(lg, s.k, renorm=s.renorm, sigmoid=s.scoring == em.SCORE_SIGMOID, bias=hl.bias,
                         groups_n=s.groups_n, groups_top=s.groups_top)
    assert np.array_equal(r["idx"], idx) and same_bits(r["gates"], gates)


def _softmax(spec):
    return spec.scoring == em.SCORE_SOFTMAX and not spec.bias_std and spec.groups_n <= 1


CASES = {
    # name: spec kwargs
    "q8_small": dict(d=1024, d_ff=512, E=8, k=2, wtype=em.Q8_0),
    "q4_small": dict(d=1024, d_ff=512, E=8, k=2, wtype=em.Q4_K),
    "q8_top4_e16": dict(d=512, d_ff=768, E=16, k=4, wtype=em.Q8_0),
    "q4_top8_e128": dict(d=2048, d_ff=768, E=128, k=8, wtype=em.Q4_K),  # config 3's shape
    "q8_odd_slices": dict(d=320, d_ff=192, E=4, k=2, wtype=em.Q8_0),    # d not a multiple of 256, 3 slices
    "q8_k_eq_e": dict(d=512, d_ff=256, E=3, k=3, wtype=em.Q8_0),        # every expert picked
    "q4_raw_gates": dict(d=1024, d_ff=512, E=8, k=2, wtype=em.Q4_K, renorm=False),
    "q8_deepseek": dict(d=1024, d_ff=512, E=16, k=4, wtype=em.Q8_0, scoring=em.SCORE_SIGMOID, bias_std=1.0,
                        groups_n=4, groups_top=2, out_scale=2.5),
    "q8_e256_k8": dict(d=1024, d_ff=256, E=256, k=8, wtype=em.Q8_0),                 # the most experts fused
    "q8_deepseek_e256": dict(d=1024, d_ff=256, E=256, k=8, wtype=em.Q8_0, scoring=em.SCORE_SIGMOID, bias_std=1.0,
                             groups_n=8, groups_top=4, out_scale=2.5),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_one_token_paths(gpu, monkeypatch, name):
    spec = em.LayerSpec(seed=31, **CASES[name])
    hl, dl = _device_layer(spec)
    for seed in (1, 2, 3):
        x = em.make_input(spec, 1, seed=seed)
        want = run_oracle(hl, x)
        ys = {}
        for path in PATHS:
            _on_path(monkeypatch, dl, path)
            print(f"one-token {name} seed={seed} path={path}", flush=True)
            y, r = _run(dl, x)
            assert np.isfinite(y).all()
            _check_routing(hl, x, r)
            if _softmax(spec):
                assert r["conflict"] == 0  # reset by the call (the scratch started as 0xff bytes)
            y2, _ = _run(dl, x)
            assert same_bits(y, y2), "not deterministic"
            ys[path] = y
            err = rel_l2(y, want)
            print(f"  rel-L2 vs oracle {err:.2e}", flush=True)
            assert err < 2e-3, err
        # the slices: the f32 summation order (Q8_0); the pack's fp16 group factors d * sc, -dmin * m (Q4_K)
        d = rel_l2(ys["slices"], ys["gemv"])
        assert d < (1e-5 if spec.wtype == em.Q8_0 else 2e-3), d


def test_without_pack_takes_gemv(gpu, monkeypatch):
    """Without a prefill pack the one-token call takes the GEMV path (the slices read the pack's tiles)."""
    monkeypatch.setenv("EMBER_MOE_SLICES", "1")
    spec = em.LayerSpec(seed=33, **CASES["q8_small"])
    hl, dl = _device_layer(spec, pack=False)
    bits = em.path(dl.desc, 1)
    assert bits & em.PATH_FUSED_ROUTE and not bits & em.PATH_SLICES, bits
    x = em.make_input(spec, 1, seed=4)
    y, r = _run(dl, x)
    _check_routing(hl, x, r)
    assert rel_l2(y, run_oracle(hl, x)) < 2e-3


@pytest.mark.parametrize("path", sorted(PATHS))
def test_conflict_poisons_output(gpu, monkeypatch, path):
    """A pick set proven from wrong fast logits (EMBER_MOE_TEST_FAST_CORRUPT: negated values under tight
    bounds) must give NaN rows and set the per-call conflict word on every one-token path."""
    spec = em.LayerSpec(seed=41, d=1024, d_ff=512, E=8, k=2, wtype=em.Q8_0)
    hl, dl = _device_layer(spec)
    x = em.make_input(spec, 1, seed=42)
    _on_path(monkeypatch, dl, path)
    y0, r0 = _run(dl, x)
    assert r0["conflict"] == 0 and np.isfinite(y0).all()
    monkeypatch.setenv("EMBER_MOE_TEST_FAST_CORRUPT", "1")
    print(f"conflict path={path}", flush=True)
    y1, r1 = _run(dl, x)
    monkeypatch.delenv("EMBER_MOE_TEST_FAST_CORRUPT")
    assert r1["conflict"] == 1 and np.isnan(y1).all()
    _check_routing(hl, x, r1)
    y2, r2 = _run(dl, x)
    assert r2["conflict"] == 0 and same_bits(y2, y0)


_mixtral = {}


def _mixtral_layer(wtype):
    if wtype not in _mixtral:
        _mixtral.clear()
        spec = em.LayerSpec(seed=0, d=4096, d_ff=14336, E=8, k=2, wtype=wtype)
        _mixtral[wtype] = _device_layer(spec)
    return _mixtral[wtype]


@pytest.mark.parametrize("wtype", [em.Q4_K, em.Q8_0])
def test_mixtral_shape_decode_call(gpu, monkeypatch, wtype):
    """Config 5's decode-shaped MoE call (Q4_K, d 4096, d_ff 14336, E 8, top-2, T = 1) and config 2's
    (Q8_0), on both one-token paths, each against the oracle."""
    hl, dl = _mixtral_layer(wtype)
    s = hl.spec
    for seed in (7, 8):
        x = em.make_input(s, 1, seed=seed)
        want = run_oracle(hl, x)
        ys = {}
        for path in PATHS:
            _on_path(monkeypatch, dl, path)
            if path == "gemv":
                assert em.path(dl.desc, 1) & em.PATH_DOWN1
            print(f"mixtral-shape {em.TYPE_NAMES[wtype]} seed={seed} path={path}", flush=True)
            y, r = _run(dl, x)
            _check_routing(hl, x, r)
            err = rel_l2(y, want)
            print(f"  rel-L2 {err:.2e}", flush=True)
            assert err < 2e-3
            ys[path] = y
