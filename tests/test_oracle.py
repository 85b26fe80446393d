"""Pins the CPU oracle (oracle/moe_oracle.cpp) before it is trusted as the parity checker.

Each check is chosen so a plausible slip (a dropped term, a wrong index, a transposed operand, a
different summation order) fails one of them:
  * golden vectors written by the reference's own code (tests/golden/make_golden.py), bit-exact;
  * the reference built in place (oracle/_ref) on fresh random inputs, bit-exact (skipped where the
    reference is absent, e.g. on the GPU box);
  * closed forms: numpy's stable argsort for the dispatch permutation, IEEE binary16 decoding,
    exact Q8_0 products, softmax identities for the gates, an FP64 brute force at the reference's
    own 1e-4 bar (tools/moe_ffn_test.cu:82-84).
"""
import hashlib
import math

import numpy as np
import pytest

import ember_moe as em
from golden_util import f32, load_cases
from oracle import oracle as O


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(both_nan | (a.view(np.uint32) == b.view(np.uint32))))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ---------------------------------------------------------------- golden vectors (reference output)


def test_golden_c1_layer_bit_exact():
    spec = em.LayerSpec(d=256, d_ff=688, E=8, k=2, wtype=em.F32, seed=0)
    hl = em.make_host_layer(spec)
    R = hl.router
    G, U, D = (hl.dequantized(n) for n in ("gate", "up", "down"))
    cases = load_cases("c1_layer.npz")
    assert len(cases) == 4
    for name, c in cases.items():
        T = int(c["T"])
        x = em.make_input(spec, T)
        # the generator must still produce the inputs the golden was written from
        assert sha(R) == str(c["sha_router"]) and sha(G) == str(c["sha_gate"]), name
        assert sha(U) == str(c["sha_up"]) and sha(D) == str(c["sha_down"]) and sha(x) == str(c["sha_x"]), name
        y = O.moe_layer(x, R, G, U, D, spec.d_ff, spec.E, spec.k, renorm=bool(c["renorm"]))
        assert same_bits(y, f32(c["out_bits"])), name


def test_golden_routing_edges_bit_exact():
    cases = load_cases("routing_edges.npz")
    assert len(cases) == 20
    for name, c in cases.items():
        y = O.moe_layer(c["x"], c["R"], c["G"], c["U"], c["D"], int(c["d_ff"]), int(c["E"]), int(c["k"]),
                        renorm=bool(c["renorm"]))
        assert same_bits(y, f32(c["out_bits"])), name


def test_golden_routed_router_bit_exact():
    cases = load_cases("routed_router.npz")
    assert len(cases) == 22
    for name, c in cases.items():
        bias = c["bias"] if c["bias"].size else None
        y = O.moe_layer(c["x"], c["R"], c["G"], c["U"], c["D"], int(c["d_ff"]), int(c["E"]), int(c["k"]),
                        renorm=bool(c["renorm"]), sigmoid=bool(c["sigmoid"]), bias=bias,
                        groups_n=int(c["groups_n"]), groups_top=int(c["groups_top"]))
        assert same_bits(y, f32(c["out_bits"])), name


def test_golden_shared_expert_bit_exact():
    cases = load_cases("shared_expert.npz")
    for name, c in cases.items():
        y = O.moe_layer(c["x"], c["R"], c["G"], c["U"], c["D"], int(c["d_ff"]), int(c["E"]), int(c["k"]),
                        renorm=True, bias=c["bias"], scale=float(c["scale"]), d_ff_sh=int(c["dsh"]),
                        Gs=c["Gs"], Us=c["Us"], Ds=c["Ds"])
        assert same_bits(y, f32(c["out_bits"])), name


def test_golden_gated_shared_expert_bit_exact():
    """qwen2moe's sigmoid-gated shared expert (graph_ir.cpp:694-705) against the reference's own ops."""
    cases = load_cases("gated_shared.npz")
    assert len(cases) == 2
    for name, c in cases.items():
        T = c["x"].shape[0]
        sg = np.empty(T, np.float32)
        y = O.moe_layer(c["x"], c["R"], c["G"], c["U"], c["D"], int(c["d_ff"]), int(c["E"]), int(c["k"]),
                        renorm=False, d_ff_sh=int(c["dsh"]), Gs=c["Gs"], Us=c["Us"], Ds=c["Ds"], Wsg=c["Wsg"],
                        sgate_out=sg)
        assert same_bits(sg, f32(c["sgate_bits"])), name
        assert same_bits(y, f32(c["out_bits"])), name
        # the gate matters: without it the output differs
        y0 = O.moe_layer(c["x"], c["R"], c["G"], c["U"], c["D"], int(c["d_ff"]), int(c["E"]), int(c["k"]),
                         renorm=False, d_ff_sh=int(c["dsh"]), Gs=c["Gs"], Us=c["Us"], Ds=c["Ds"])
        assert not same_bits(y0, y)


def test_golden_dequant_kats():
    z = np.load(f"{__import__('golden_util').GOLDEN}/dequant_kat.npz")
    fp16 = np.array([O.ora().oracle_fp16_to_fp32(h) for h in range(65536)], np.float32)
    assert same_bits(fp16, f32(z["fp16_bits"]))
    nb = z["q8_raw"].shape[0]
    assert same_bits(O.dequant(em.Q8_0, z["q8_raw"], nb * 32), f32(z["q8_out_bits"]))
    assert same_bits(O.dequant(em.Q4_K, z["q4_raw"], nb * 256), f32(z["q4_out_bits"]))


# ---------------------------------------------------------------- closed forms


def test_fp16_matches_ieee_half():
    codes = np.arange(65536, dtype=np.uint16)
    ieee = codes.view(np.float16).astype(np.float32)
    ours = np.array([O.ora().oracle_fp16_to_fp32(int(h)) for h in codes], np.float32)
    assert same_bits(ours, ieee)


def test_q8_0_dequant_closed_form():
    rng = np.random.default_rng(1)
    nb = 64
    raw = rng.integers(0, 256, size=(nb, 34), dtype=np.uint8)
    d = (rng.standard_normal(nb) * 0.01).astype(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    q = raw[:, 2:].view(np.int8).astype(np.float32)
    want = (d.astype(np.float32)[:, None] * q).reshape(-1)  # one exact-rounded product each
    assert same_bits(O.dequant(em.Q8_0, raw, nb * 32), want)


def test_q4_k_dequant_layout():
    """A block built from known 6-bit scales/mins and nibbles decodes to d*sc*q - dmin*m per group,
    with group g's nibble of element l at byte 32*(g//2) + l, low half for even g."""
    rng = np.random.default_rng(2)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    q = rng.integers(0, 16, 256)
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.25], np.float16).view(np.uint8)
    for j in range(4):
        blk[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    for c in range(4):
        for l in range(32):
            blk[16 + 32 * c + l] = q[64 * c + l] | (q[64 * c + 32 + l] << 4)
    want = np.array([np.float32(0.5 * sc[g]) * np.float32(q[32 * g + l]) - np.float32(0.25 * mn[g])
                     for g in range(8) for l in range(32)], np.float32)
    assert same_bits(O.dequant(em.Q4_K, blk, 256), want)


def test_bf16_and_f32_dequant():
    rng = np.random.default_rng(3)
    v = rng.standard_normal(1000).astype(np.float32)
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    assert same_bits(O.dequant(em.BF16, bf, 1000), (bf.astype(np.uint32) << 16).view(np.float32))
    assert same_bits(O.dequant(em.F32, v, 1000), v)


def _dot_closed_form(a, b):
    n = len(a)
    n8 = n - n % 8
    lanes = [0.0] * 8
    for i in range(n8):
        lanes[i % 8] += float(a[i]) * float(b[i])
    tail = 0.0
    for i in range(n8, n):
        tail += float(a[i]) * float(b[i])
    return ((lanes[0] + lanes[1]) + (lanes[2] + lanes[3])) + ((lanes[4] + lanes[5]) + (lanes[6] + lanes[7])) + tail


@pytest.mark.parametrize("n", [1, 7, 8, 9, 64, 100, 257])
def test_dot_fixed_order(n):
    """cpu_dot.h:12-21: Python floats are binary64 and each f32 x f32 product is exact in binary64,
    so this loop is the eight-chain sum itself; a different lane count or tree order changes bits."""
    rng = np.random.default_rng(n)
    a = (rng.standard_normal(n) * 10 ** rng.uniform(-3, 3, n)).astype(np.float32)
    b = (rng.standard_normal(n) * 10 ** rng.uniform(-3, 3, n)).astype(np.float32)
    assert O.dot(a, b) == _dot_closed_form(a, b)
    assert abs(O.dot(a, b) - math.fsum(float(x) * float(y) for x, y in zip(a, b))) <= 1e-12 * np.sum(np.abs(a * b)) + 1e-300


def test_dispatch_is_stable_sort():
    rng = np.random.default_rng(4)
    for T, k, E in ((1, 2, 8), (37, 8, 128), (64, 6, 64), (5, 3, 4)):
        idx = np.stack([np.sort(rng.choice(E, size=k, replace=False)) for _ in range(T)]).astype(np.int32)
        offsets, perm = O.dispatch(idx, E)
        flat = idx.reshape(-1)
        want = np.argsort(flat, kind="stable")
        assert np.array_equal(perm, want)
        assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))


def test_route_softmax_identities():
    rng = np.random.default_rng(6)
    logits = (rng.standard_normal((200, 16)) * 3).astype(np.float32)
    for renorm in (True, False):
        idx, gates = O.route(logits, 4, renorm=renorm)
        for t in range(200):
            r = logits[t].astype(np.float64)
            order = sorted(range(16), key=lambda e: (-r[e], e))[:4]
            assert list(idx[t]) == sorted(order)
            pool = r[sorted(order)] if renorm else r
            p = np.exp(r[idx[t]] - pool.max()) / np.exp(pool - pool.max()).sum()
            # r - mx is a float subtraction in the reference: relative error <= |r - mx| * 2^-24
            assert np.allclose(gates[t], p, rtol=2e-6, atol=0)
        if renorm:
            assert np.allclose(gates.sum(1), 1.0, atol=1e-6)


def test_route_ties_keep_lower_index():
    logits = np.array([[1.0, 3.0, 3.0, 0.5, 3.0, -1.0]], np.float32)
    idx, _ = O.route(logits, 2)
    assert list(idx[0]) == [1, 2]
    idx, _ = O.route(np.zeros((1, 8), np.float32), 3)
    assert list(idx[0]) == [0, 1, 2]


def test_layer_fp64_bruteforce():
    """tools/moe_ffn_test.cu's procedure: E 8, k 2, d 96, d_ff 160, weights and inputs scaled normals,
    compared with a float64 evaluation at max |err| < 1e-4."""
    rng = np.random.default_rng(3)
    E, k, d, d_ff = 8, 2, 96, 160
    R = (rng.standard_normal((E, d)) * 0.3).astype(np.float32)
    G = (rng.standard_normal((E, d_ff, d)) * 0.3).astype(np.float32)
    U = (rng.standard_normal((E, d_ff, d)) * 0.3).astype(np.float32)
    D = (rng.standard_normal((E, d, d_ff)) * 0.3).astype(np.float32)
    for renorm in (True, False):
        for T in (1, 2, 5, 16, 17, 40):
            x = (rng.standard_normal((T, d)) * 0.9).astype(np.float32)
            y = O.moe_layer(x, R, G, U, D, d_ff, E, k, renorm=renorm)
            ref = np.zeros((T, d))
            for t in range(T):
                r = R.astype(np.float64) @ x[t].astype(np.float64)
                sel = sorted(sorted(range(E), key=lambda e: (-r[e], e))[:k])
                pool = r[sel] if renorm else r
                z = np.exp(pool - pool.max()).sum()
                for e in sel:
                    gv = G[e].astype(np.float64) @ x[t]
                    uv = U[e].astype(np.float64) @ x[t]
                    h = gv / (1 + np.exp(-gv)) * uv
                    ref[t] += np.exp(r[e] - pool.max()) / z * (D[e].astype(np.float64) @ h)
            assert np.max(np.abs(y - ref)) < 1e-4, (renorm, T)


# ---------------------------------------------------------------- the reference built in place

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (reference absent)")


@needs_ref
def test_ref_dot_bits():
    rng = np.random.default_rng(9)
    for n in (3, 8, 33, 256, 688, 4096):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        r = O.ref()
        assert O.dot(a, b) == r.ref_dot_f32_f64(a.ctypes.data, b.ctypes.data, n)
        assert O.dot(a, b) == r.ref_dot_f32_f64_portable(a.ctypes.data, b.ctypes.data, n)


@needs_ref
@pytest.mark.parametrize("d,d_ff,E,k", [(20, 36, 6, 2), (64, 96, 16, 4), (33, 17, 5, 5), (24, 8, 3, 4)])
def test_ref_layer_random(d, d_ff, E, k):
    rng = np.random.default_rng(d * 1000 + d_ff)
    R = (rng.standard_normal((E, d)) * 0.5).astype(np.float32)
    G = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    U = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    D = (rng.standard_normal((E, d, d_ff)) * 0.2).astype(np.float32)
    x = rng.standard_normal((7, d)).astype(np.float32)
    bias = (rng.standard_normal(E) * 2).astype(np.float32)
    for renorm in (0, 1):
        out = np.empty((7, d), np.float32)
        O.ref().ref_moe_ffn_f32(x.ctypes.data, 7, d, d_ff, E, k, R.ctypes.data, G.ctypes.data, U.ctypes.data,
                                D.ctypes.data, out.ctypes.data, renorm)
        assert same_bits(O.moe_layer(x, R, G, U, D, d_ff, E, k, renorm=bool(renorm)), out)
        for sigmoid in (0, 1):
            O.ref().ref_moe_ffn_routed_f32(x.ctypes.data, 7, d, d_ff, E, k, R.ctypes.data, G.ctypes.data,
                                           U.ctypes.data, D.ctypes.data, out.ctypes.data, renorm, sigmoid,
                                           bias.ctypes.data, 1, 1)
            y = O.moe_layer(x, R, G, U, D, d_ff, E, k, renorm=bool(renorm), sigmoid=bool(sigmoid), bias=bias)
            assert same_bits(y, out)


@needs_ref
def test_ref_dequant_random_blocks():
    rng = np.random.default_rng(10)
    nb = 128
    q8 = rng.integers(0, 256, size=(nb, 34), dtype=np.uint8)
    q4 = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    o8 = np.empty(nb * 32, np.float32)
    o4 = np.empty(nb * 256, np.float32)
    O.ref().ref_dequant_q8_0(q8.ctypes.data, nb, o8.ctypes.data)
    O.ref().ref_dequant_q4_k(q4.ctypes.data, nb, o4.ctypes.data)
    assert same_bits(O.dequant(em.Q8_0, q8, nb * 32), o8)
    assert same_bits(O.dequant(em.Q4_K, q4, nb * 256), o4)
