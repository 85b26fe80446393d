"""GPU parity of the router logits, routing and dispatch (bit-exact against the oracle).

Bar: logits, expert indices, gate values and the dispatch permutation must be bit-identical to the
reference's CPU path given the same inputs (utils.cpp:704-836; the permutation against the stable
sort of the oracle)."""
import numpy as np
import pytest

import ember_moe as em
from gpu_util import same_bits
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("T,d,E", [(1, 4096, 8), (8, 4096, 8), (3, 100, 8), (64, 2048, 128), (257, 2048, 64), (2048, 4096, 8),
                                   (512, 2048, 128), (300, 256, 100), (520, 2048, 64), (2050, 512, 16),
                                   (40, 256, 8), (31, 20, 5), (1500, 520, 200), (300, 2052, 24), (9, 100, 16), (100, 36, 12),
                                   (4, 64, 16)])
def test_router_logits_bit_exact(gpu, T, d, E):
    import torch

    rng = np.random.default_rng(T * 7 + E)
    x = rng.standard_normal((T, d)).astype(np.float32)
    R = (rng.standard_normal((E, d)) / np.sqrt(d)).astype(np.float32)
    lg = torch.empty((T, E), dtype=torch.float32, device="cuda")
    print(f"router_logits T={T} d={d} E={E}", flush=True)
    assert em.router_logits(_dev(x), T, d, E, _dev(R), lg) == 0
    torch.cuda.synchronize()
    assert same_bits(lg.cpu().numpy(), O.router_logits(x, R))


def _route_gpu(logits, k, renorm=True, scoring=em.SCORE_SOFTMAX, bias=None, groups_n=1, groups_top=1, scratch=None):
    import torch

    T, E = logits.shape
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    gates = torch.empty((T, k), dtype=torch.float32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    perm = torch.full((T * k,), -1, dtype=torch.int32, device="cuda")
    if scratch is None:
        scratch = torch.empty(em.route_scratch_bytes(T, E, k), dtype=torch.uint8, device="cuda")
    s = em.route(_dev(logits), T, E, k, renorm, scoring, None if bias is None else _dev(bias), groups_n, groups_top,
                 idx, gates, offsets, perm, scratch)
    assert s == 0, em.strerror(s)
    torch.cuda.synchronize()
    return idx.cpu().numpy(), gates.cpu().numpy(), offsets.cpu().numpy(), perm.cpu().numpy()


def _edge_logits(rng, T, E):
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    lg[0, :] = 0.0                                   # all tied
    if T > 1:
        lg[1, 1::3] = lg[1, 0]                       # a tie class
    if T > 2:
        lg[2, E // 2] = np.inf
        lg[2, 0] = -np.inf
    if T > 3:
        lg[3, 2] = np.nan                            # serial path
    if T > 4:
        lg[4, :] = -np.inf
    if T > 5 and E > 4:
        lg[5, 3] = -0.0
        lg[5, 4] = 0.0
    if T > 6:
        lg[6] = np.round(lg[6])                      # many small-integer ties
    return lg


@pytest.mark.parametrize("T,E,k", [(1, 8, 2), (8, 8, 2), (13, 64, 6), (128, 128, 8), (7, 200, 5), (9, 16, 16),
                                   (4096, 128, 8), (2048, 8, 2), (6, 4, 7), (3, 256, 8), (40, 256, 8), (5, 300, 10),
                                   (2, 512, 4), (33, 512, 12), (1000, 256, 8), (1025, 64, 8), (700, 16, 17),
                                   (64, 8, 2), (64, 128, 8), (57, 32, 4), (16, 8, 2), (65, 128, 8)])
@pytest.mark.parametrize("renorm", [True, False])
def test_route_softmax_bit_exact(gpu, T, E, k, renorm):
    rng = np.random.default_rng(T * 131 + E * 7 + k)
    lg = _edge_logits(rng, T, E)
    print(f"route T={T} E={E} k={k} renorm={renorm}", flush=True)
    idx, gates, offsets, perm = _route_gpu(lg, k, renorm)
    widx, wgates = O.route(lg, k, renorm=renorm)
    assert np.array_equal(idx, widx)
    assert same_bits(gates, wgates)
    woff, wperm = O.dispatch(widx, E)
    assert np.array_equal(offsets, woff)
    n = int(woff[-1])
    assert np.array_equal(perm[:n], wperm[:n])


@pytest.mark.parametrize("sigmoid", [False, True])
@pytest.mark.parametrize("use_bias", [False, True])
@pytest.mark.parametrize("groups", [(1, 1), (4, 2), (8, 3)])
def test_route_deepseek_bit_exact(gpu, sigmoid, use_bias, groups):
    if not sigmoid and not use_bias and groups[0] == 1:
        pytest.skip("plain softmax is covered above")
    rng = np.random.default_rng(17)
    T, E, k = 37, 64, 6
    lg = _edge_logits(rng, T, E)
    bias = (rng.standard_normal(E) * 2).astype(np.float32) if use_bias else None
    for renorm in (True, False):
        idx, gates, offsets, perm = _route_gpu(lg, k, renorm, em.SCORE_SIGMOID if sigmoid else em.SCORE_SOFTMAX, bias,
                                               *groups)
        widx, wgates = O.route(lg, k, renorm=renorm, sigmoid=sigmoid, bias=bias, groups_n=groups[0],
                               groups_top=groups[1])
        assert np.array_equal(idx, widx)
        assert same_bits(gates, wgates)
        woff, wperm = O.dispatch(widx, E)
        assert np.array_equal(offsets, woff)
        assert np.array_equal(perm[:woff[-1]], wperm[:woff[-1]])


def test_route_reuses_scratch(gpu):
    """One scratch buffer, first filled with 0xff bytes, serves routing calls of several sizes in a row
    (one-block fused routing + dispatch at 8 tokens or fewer, separate route and dispatch launches above):
    each call's picks, gates and dispatch match the oracle, whatever an earlier call left in the scratch."""
    import torch

    rng = np.random.default_rng(5)
    E, k = 64, 6
    scratch = torch.full((em.route_scratch_bytes(64, E, k),), 0xFF, dtype=torch.uint8, device="cuda")
    for T in (64, 17, 64, 9, 40, 8, 33):
        lg = _edge_logits(rng, T, E)
        print(f"route reuse T={T}", flush=True)
        idx, gates, offsets, perm = _route_gpu(lg, k, True, scratch=scratch)
        widx, wgates = O.route(lg, k, renorm=True)
        assert np.array_equal(idx, widx) and same_bits(gates, wgates)
        woff, wperm = O.dispatch(widx, E)
        assert np.array_equal(offsets, woff)
        assert np.array_equal(perm[:woff[-1]], wperm[:woff[-1]])


def test_route_dense_sweep_random(gpu):
    """Many random rows: gates through exp / division / rounding match glibc's bits everywhere."""
    rng = np.random.default_rng(99)
    for E, k in ((8, 2), (128, 8), (64, 6)):
        lg = (rng.standard_normal((8192, E)) * rng.uniform(0.1, 30)).astype(np.float32)
        for renorm in (True, False):
            idx, gates, _, _ = _route_gpu(lg, k, renorm)
            widx, wgates = O.route(lg, k, renorm=renorm)
            assert np.array_equal(idx, widx)
            assert same_bits(gates, wgates)
