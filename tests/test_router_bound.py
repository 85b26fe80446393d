"""The proven-picks router's error bound (moe_router_fast.hip), restated in numpy and held against the
oracle's exact logits (the reference's FP64 eight-chain dot, utils.cpp:707 / cpu_dot.h:12-21): rows
scaled by a power of two into (63.5, 127], written as two int8 planes a1 = rint(X), a2 = rint(254 (X - a1))
(f32 arithmetic, as the kernel does it), fast = s_x s_r (254^2 a1.b1 + 254 (a1.b2 + a2.b1) + a2.b2) / 254^2,
and B = s_x s_r ((sum |X| + sum |R|) kEps + d kEps^2) plus the chains' and the f32 rounding terms. Every
logit must lie in [fast - B, fast + B], on seeded normals and on rows built to stress the bound; the bound
must also be useful (far below the logits' spread), or the router would prune nothing."""
import numpy as np
import pytest

from oracle import oracle as O

EPS = 1.0 / 508.0 + 2.0 ** -25


def _quant(v):
    mx = np.abs(v).max(axis=1)
    f, ex = np.frexp(mx.astype(np.float64))
    q = np.where(f * 128 <= 127, ex - 7, ex - 6).astype(np.int32)
    q = np.where(mx > 0, q, 0)
    X = np.ldexp(v.astype(np.float32), -q[:, None]).astype(np.float32)
    a1 = np.rint(X)
    a2 = np.rint(((X - a1) * np.float32(254)).astype(np.float32))
    SX = np.abs(X.astype(np.float64)).sum(axis=1) * (1 + 2.0 ** -20) + v.shape[1] * 2.0 ** -140
    return a1.astype(np.float64), a2.astype(np.float64), np.ldexp(1.0, q), SX


def _bounds(x, R):
    d = x.shape[1]
    a1, a2, sx, SX = _quant(x)
    b1, b2, sr, SR = _quant(R)
    F = 64516.0 * (a1 @ b1.T) + 254.0 * (a1 @ b2.T + a2 @ b1.T) + (a2 @ b2.T)  # integers below 2^53: exact
    ss = sx[:, None] * sr[None, :]
    fast = F * ss / 64516.0
    B = ss * ((SX[:, None] + SR[None, :]) * EPS + d * EPS * EPS)
    B += ss * 127 * np.minimum(SX[:, None], SR[None, :]) * ((d / 8 + 8) * 1.125 * 2.0 ** -53)
    B = B * (1 + 2.0 ** -40) + np.abs(fast) * 2.0 ** -48
    B += (np.abs(fast) + B) * 2.0 ** -23 + 2.0 ** -148
    return fast - B, fast + B


@pytest.mark.parametrize("kind", ["normal", "scaled", "outlier", "sparse", "near"])
@pytest.mark.parametrize("T,d,E", [(96, 2048, 128), (64, 4096, 8), (70, 96, 200)])
def test_bound_brackets_exact_logits(T, d, E, kind):
    rng = np.random.default_rng(T + d + E)
    x = rng.standard_normal((T, d)).astype(np.float32)
    R = (rng.standard_normal((E, d)) / np.sqrt(d)).astype(np.float32)
    if kind == "scaled":
        x *= np.exp2(rng.integers(-60, 61, size=(T, 1))).astype(np.float32)
        R *= np.exp2(rng.integers(-30, 31, size=(E, 1))).astype(np.float32)
    elif kind == "outlier":
        x[np.arange(T), rng.integers(0, d, size=T)] *= 1e4
    elif kind == "sparse":
        x[rng.random((T, d)) < 0.97] = 0.0
        x[0] = 0.0
    elif kind == "near":
        R[1:6] = R[0]
        R[1:6, 0] = np.nextafter(R[0, 0], np.float32(np.inf))
    L, U = _bounds(x, R)
    lg = O.router_logits(x, R).astype(np.float64)
    assert np.all(L <= lg) and np.all(lg <= U)
    if kind == "normal":
        width = (U - L).mean()
        assert width < 0.02 * lg.std(), width  # useful: a small fraction of the logits' spread
