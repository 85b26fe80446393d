"""Writes the golden vectors under tests/golden/ from the reference's own CPU MoE code.

Runs in the build container only: it loads oracle/_ref/libref_moe.so, which oracle/Makefile compiles
from /root/reference/{utils,quantization,logger}.cpp with a C-ABI harness (oracle/ref_harness.cpp).
Inputs come from this project's seeded generator (ember_moe.normal) or are small explicit arrays;
each fixture stores its inputs (or their generator parameters plus SHA-256), and the reference's
outputs as raw float bits. Nothing from /root/reference is stored.

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "ember.cpp_amd")]

import ember_moe as em  # noqa: E402
from oracle import oracle as O  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def vp(a):
    return None if a is None else a.ctypes.data


def ref_layer(x, R, G, U, D, d_ff, E, k, renorm, sigmoid=False, bias=None, groups_n=1, groups_top=1):
    T, d = x.shape
    out = np.empty((T, d), np.float32)
    if not sigmoid and bias is None and groups_n <= 1:
        O.ref().ref_moe_ffn_f32(x.ctypes.data, T, d, d_ff, E, k, R.ctypes.data, G.ctypes.data, U.ctypes.data,
                                D.ctypes.data, out.ctypes.data, int(renorm))
    else:
        O.ref().ref_moe_ffn_routed_f32(x.ctypes.data, T, d, d_ff, E, k, R.ctypes.data, G.ctypes.data,
                                       U.ctypes.data, D.ctypes.data, out.ctypes.data, int(renorm), int(sigmoid),
                                       vp(bias), groups_n, groups_top)
    return out


def c1_cases():
    """d 256, E 8, top-2, d_ff 688, F32, seed 0; T = 1 and 64; renorm and raw."""
    out = {}
    spec = em.LayerSpec(d=256, d_ff=688, E=8, k=2, wtype=em.F32, seed=0)
    hl = em.make_host_layer(spec)
    R = hl.router
    G, U, D = (hl.dequantized(n) for n in ("gate", "up", "down"))
    for T in (1, 64):
        x = em.make_input(spec, T)
        for renorm in (1, 0):
            y = ref_layer(x, R, G, U, D, spec.d_ff, spec.E, spec.k, renorm)
            key = f"c1_T{T}_{'renorm' if renorm else 'raw'}"
            out[key] = dict(T=T, renorm=renorm, sha_router=sha(R), sha_gate=sha(G), sha_up=sha(U), sha_down=sha(D),
                            sha_x=sha(x), out_bits=y.view(np.uint32))
    return out


def routing_edge_cases():
    """Small layers whose router produces exact ties, +-inf and NaN logits (d 16, d_ff 32, E 8, k 3),
    and a k > E layer. Inputs stored whole."""
    rng = np.random.default_rng(7)
    d, d_ff, E = 16, 32, 8
    cases = {}
    G = (rng.standard_normal((E, d_ff, d)) * 0.3).astype(np.float32)
    U = (rng.standard_normal((E, d_ff, d)) * 0.3).astype(np.float32)
    D = (rng.standard_normal((E, d, d_ff)) * 0.3).astype(np.float32)
    x = (rng.standard_normal((6, d)) * 1.5).astype(np.float32)
    base = (rng.standard_normal((E, d)) * 0.5).astype(np.float32)
    variants = {}
    R = base.copy(); R[5] = R[2]; R[6] = R[2]; variants["ties"] = R          # experts 2, 5, 6 tie
    R = base.copy(); R[3] = 0; R[4] = 0; variants["zero_ties"] = R           # two zero logits
    R = base.copy(); R[1, 0] = np.inf; variants["inf"] = R                   # +inf / -inf / NaN by x's sign
    R = base.copy(); R[7, :] = np.nan; variants["nan_row"] = R               # one NaN logit per token
    R = base.copy(); R[0, 3] = np.float32(1e30); R[4, 3] = np.float32(-1e30); variants["huge"] = R
    for name, R in variants.items():
        for renorm in (1, 0):
            for k in (3, 8):
                y = ref_layer(x, R, G, U, D, d_ff, E, k, renorm)
                cases[f"edge_{name}_k{k}_{'renorm' if renorm else 'raw'}"] = dict(
                    x=x, R=R, G=G, U=U, D=D, d_ff=d_ff, E=E, k=k, renorm=renorm, out_bits=y.view(np.uint32))
    return cases


def routed_cases():
    """moe_ffn_routed_f32_cpu (DeepSeek-V3 router): sigmoid / softmax scores, a selection bias,
    groups; d 32, d_ff 48, E 16. Inputs stored whole."""
    rng = np.random.default_rng(11)
    d, d_ff, E = 32, 48, 16
    G = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    U = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    D = (rng.standard_normal((E, d, d_ff)) * 0.2).astype(np.float32)
    R = (rng.standard_normal((E, d)) / np.sqrt(d)).astype(np.float32)
    x = rng.standard_normal((9, d)).astype(np.float32)
    bias = (rng.standard_normal(E) * 2.0).astype(np.float32)
    cases = {}
    for sigmoid in (0, 1):
        for use_bias in (0, 1):
            for groups_n, groups_top, k in ((1, 1, 4), (4, 2, 4), (8, 3, 6)):
                if not sigmoid and not use_bias and groups_n == 1:
                    continue
                for renorm in (1, 0):
                    b = bias if use_bias else None
                    y = ref_layer(x, R, G, U, D, d_ff, E, k, renorm, sigmoid, b, groups_n, groups_top)
                    cases[f"routed_s{sigmoid}_b{use_bias}_g{groups_n}_{groups_top}_k{k}_{'renorm' if renorm else 'raw'}"] = dict(
                        x=x, R=R, G=G, U=U, D=D, bias=bias if use_bias else np.zeros(0, np.float32), d_ff=d_ff, E=E,
                        k=k, renorm=renorm, sigmoid=sigmoid, groups_n=groups_n, groups_top=groups_top,
                        out_bits=y.view(np.uint32))
    return cases


def shared_cases():
    """The IR's deepseek2 FFN (graph_ir.cpp:919-928): f = moe_ffn(h) [* scale]; sf = linear(down_sh,
    silu(linear(gate_sh, h)) * linear(up_sh, h)); f = f + sf — composed from the reference's own
    moe_ffn_routed_f32_cpu, matmul_f32_f32_batch_cpu and silu_cpu."""
    rng = np.random.default_rng(13)
    d, d_ff, E, k, dsh, T = 32, 48, 16, 4, 96, 5
    G = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    U = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    D = (rng.standard_normal((E, d, d_ff)) * 0.2).astype(np.float32)
    R = (rng.standard_normal((E, d)) / np.sqrt(d)).astype(np.float32)
    Gs = (rng.standard_normal((dsh, d)) * 0.2).astype(np.float32)
    Us = (rng.standard_normal((dsh, d)) * 0.2).astype(np.float32)
    Ds = (rng.standard_normal((d, dsh)) * 0.2).astype(np.float32)
    x = rng.standard_normal((T, d)).astype(np.float32)
    bias = (rng.standard_normal(E) * 2.0).astype(np.float32)
    cases = {}
    for scale in (1.0, 2.5):
        f = ref_layer(x, R, G, U, D, d_ff, E, k, 1, 0, bias, 1, 1)
        if scale != 1.0:
            f = (f * np.float32(scale) + np.float32(0.0)).astype(np.float32)
        sg = np.empty((T, dsh), np.float32); su = np.empty((T, dsh), np.float32); sf = np.empty((T, d), np.float32)
        O.ref().ref_matmul_f32_batch(Gs.ctypes.data, x.ctypes.data, sg.ctypes.data, T, dsh, d)
        O.ref().ref_matmul_f32_batch(Us.ctypes.data, x.ctypes.data, su.ctypes.data, T, dsh, d)
        sgs = np.empty_like(sg)
        O.ref().ref_silu(sg.ctypes.data, sgs.ctypes.data, sg.size)
        sgu = (sgs * su).astype(np.float32)
        O.ref().ref_matmul_f32_batch(Ds.ctypes.data, sgu.ctypes.data, sf.ctypes.data, T, d, dsh)
        y = (f + sf).astype(np.float32)
        cases[f"shared_scale{scale}"] = dict(x=x, R=R, G=G, U=U, D=D, Gs=Gs, Us=Us, Ds=Ds, bias=bias, d_ff=d_ff, E=E,
                                             k=k, dsh=dsh, scale=scale, out_bits=y.view(np.uint32))
    return cases


def gated_shared_cases():
    """qwen2moe's FFN in the IR (graph_ir.cpp:694-705): f = moe_ffn(h2) with raw gates; sf = linear(down_sh,
    silu(linear(gate_sh, h2)) * linear(up_sh, h2)); sgate = sigmoid(linear(ffn_gate_inp_shexp, h2));
    sf = mul_col(sf, sgate); f = f + sf — composed from the reference's own moe_ffn_f32_cpu,
    matmul_f32_f32_batch_cpu, silu_cpu, and graph_ir_ops.cpp's sigmoid and mul_col."""
    rng = np.random.default_rng(17)
    d, d_ff, E, k, dsh, T = 32, 48, 16, 4, 64, 7
    G = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    U = (rng.standard_normal((E, d_ff, d)) * 0.2).astype(np.float32)
    D = (rng.standard_normal((E, d, d_ff)) * 0.2).astype(np.float32)
    R = (rng.standard_normal((E, d)) / np.sqrt(d)).astype(np.float32)
    Gs = (rng.standard_normal((dsh, d)) * 0.2).astype(np.float32)
    Us = (rng.standard_normal((dsh, d)) * 0.2).astype(np.float32)
    Ds = (rng.standard_normal((d, dsh)) * 0.2).astype(np.float32)
    x = rng.standard_normal((T, d)).astype(np.float32)
    cases = {}
    for wscale in (0.3, 3.0):  # sigmoid near its middle, and saturating
        Wsg = (rng.standard_normal(d) * wscale / np.sqrt(d)).astype(np.float32)
        f = ref_layer(x, R, G, U, D, d_ff, E, k, 0)
        sg = np.empty((T, dsh), np.float32); su = np.empty((T, dsh), np.float32); sf = np.empty((T, d), np.float32)
        O.ref().ref_matmul_f32_batch(Gs.ctypes.data, x.ctypes.data, sg.ctypes.data, T, dsh, d)
        O.ref().ref_matmul_f32_batch(Us.ctypes.data, x.ctypes.data, su.ctypes.data, T, dsh, d)
        sgs = np.empty_like(sg)
        O.ref().ref_silu(sg.ctypes.data, sgs.ctypes.data, sg.size)
        sgu = (sgs * su).astype(np.float32)
        O.ref().ref_matmul_f32_batch(Ds.ctypes.data, sgu.ctypes.data, sf.ctypes.data, T, d, dsh)
        gl = np.empty((T, 1), np.float32)
        O.ref().ref_matmul_f32_batch(Wsg.ctypes.data, x.ctypes.data, gl.ctypes.data, T, 1, d)
        gate = np.empty_like(gl)
        O.ref().ref_sigmoid(gl.ctypes.data, gate.ctypes.data, gl.size)
        sfg = np.empty_like(sf)
        O.ref().ref_mul_col(sf.ctypes.data, gate.ctypes.data, sfg.ctypes.data, T, d)
        y = (f + sfg).astype(np.float32)
        cases[f"gated_w{wscale}"] = dict(x=x, R=R, G=G, U=U, D=D, Gs=Gs, Us=Us, Ds=Ds, Wsg=Wsg, d_ff=d_ff, E=E, k=k,
                                         dsh=dsh, sgate_bits=gl.reshape(T).view(np.uint32),
                                         out_bits=y.view(np.uint32))
    return cases


def dequant_kats():
    """fp16 -> f32 for all 65536 codes; Q8_0 and Q4_K blocks with random payloads (including
    negative, subnormal, Inf/NaN fp16 scales) through the reference's block dequantizers."""
    rng = np.random.default_rng(5)
    fp16 = np.array([O.ref().ref_fp16_to_fp32(h) for h in range(65536)], np.float32)
    nb = 256
    q8 = rng.integers(0, 256, size=(nb, 34), dtype=np.uint8)
    scales = rng.standard_normal(nb).astype(np.float16).view(np.uint16)
    scales[:8] = [0x0000, 0x8000, 0x0001, 0x03ff, 0x7c00, 0xfc00, 0x7e00, 0xbc00]
    q8[:, 0] = scales & 0xff
    q8[:, 1] = scales >> 8
    q8_out = np.empty(nb * 32, np.float32)
    O.ref().ref_dequant_q8_0(q8.ctypes.data, nb, q8_out.ctypes.data)
    q4 = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    dd = (np.abs(rng.standard_normal((nb, 2))) * 0.01).astype(np.float16).view(np.uint16)
    dd[:4, 0] = [0x0001, 0x0000, 0x3c00, 0x8400]
    q4[:, 0] = dd[:, 0] & 0xff; q4[:, 1] = dd[:, 0] >> 8
    q4[:, 2] = dd[:, 1] & 0xff; q4[:, 3] = dd[:, 1] >> 8
    q4_out = np.empty(nb * 256, np.float32)
    O.ref().ref_dequant_q4_k(q4.ctypes.data, nb, q4_out.ctypes.data)
    return dict(fp16_bits=fp16.view(np.uint32), q8_raw=q8, q8_out_bits=q8_out.view(np.uint32), q4_raw=q4,
                q4_out_bits=q4_out.view(np.uint32))


def main(only=None):
    if not O.ref_available():
        O.build(ref=True)
    assert O.ref_available(), "oracle/_ref/libref_moe.so could not be built (is /root/reference present?)"

    def save(name, cases):
        # Arrays shared by several cases are stored once under "blob/<sha>", and a case's field
        # holds the string "@<sha>" (see tests/golden_util.py).
        flat, blobs = {}, {}
        for key, val in cases.items():
            for f, v in val.items():
                v = np.asarray(v)
                if v.size > 64:
                    h = sha(v)[:16]
                    blobs[h] = v
                    flat[f"{key}/{f}"] = np.asarray("@" + h)
                else:
                    flat[f"{key}/{f}"] = v
        for h, v in blobs.items():
            flat[f"blob/{h}"] = v
        np.savez_compressed(os.path.join(HERE, name), **flat)
        print(name, len(cases), "cases")

    sets = {"c1_layer.npz": c1_cases, "routing_edges.npz": routing_edge_cases, "routed_router.npz": routed_cases,
            "shared_expert.npz": shared_cases, "gated_shared.npz": gated_shared_cases}
    for name, fn in sets.items():
        if only is None or name in only:
            save(name, fn())
    if only is None or "dequant_kat.npz" in only:
        kats = dequant_kats()
        np.savez_compressed(os.path.join(HERE, "dequant_kat.npz"), **kats)
        print("dequant_kat.npz")


if __name__ == "__main__":
    main(set(sys.argv[1:]) or None)
