"""ORACLE — TEST INFRASTRUCTURE ONLY.

ctypes access to the CPU parity oracle (liboracle.so, the restatement in moe_oracle.cpp) and, where it
was built in this container, to oracle/_ref/libref_moe.so (the reference's own utils.cpp /
quantization.cpp compiled in place). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product path never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_ora = None
_ref = None


def build(ref: bool = True) -> None:
    """Builds liboracle.so (and _ref/libref_moe.so when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"] + (["ref"] if ref else []), check=True)


def _vp(a):
    return None if a is None else a.ctypes.data


def ora() -> ctypes.CDLL:
    global _ora
    if _ora is None:
        p = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(p):
            build(ref=False)
        L = ctypes.CDLL(p)
        vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.oracle_dot_f32_f64.argtypes = [vp, vp, i]
        L.oracle_dot_f32_f64.restype = ctypes.c_double
        L.oracle_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.oracle_fp16_to_fp32.restype = f
        L.oracle_dequant.argtypes = [i, vp, ctypes.c_size_t, ctypes.c_size_t, vp]
        L.oracle_dequant.restype = i
        L.oracle_router_logits.argtypes = [vp, i, i, i, vp, vp]
        L.oracle_route.argtypes = [vp, i, i, i, i, i, vp, i, i, vp, vp]
        L.oracle_route.restype = i
        L.oracle_dispatch.argtypes = [vp, i, i, i, vp, vp]
        L.oracle_moe_layer.argtypes = [vp, i, i, i, i, i, i, i, vp, i, i, f, vp, vp, vp, vp, i, vp, vp, vp, vp, i]
        L.oracle_moe_layer_gated.argtypes = [vp, i, i, i, i, i, i, i, vp, i, i, f, vp, vp, vp, vp, i, vp, vp, vp, vp,
                                             vp, vp, i]
        _ora = L
    return _ora


def ref_available() -> bool:
    return os.path.exists(os.path.join(HERE, "_ref", "libref_moe.so"))


_ref_gguf = None


def ref_gguf_available() -> bool:
    return os.path.exists(os.path.join(HERE, "_ref", "libref_gguf.so"))


def ref_gguf_dump(path: str):
    """The reference's load_gguf_meta on `path` (oracle/_ref/libref_gguf.so): (0, text) on success,
    (-1, exception message) when the reference rejects the file."""
    global _ref_gguf
    if _ref_gguf is None:
        L = ctypes.CDLL(os.path.join(HERE, "_ref", "libref_gguf.so"))
        L.ref_gguf_dump.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
        L.ref_gguf_dump.restype = ctypes.c_int
        _ref_gguf = L
    cap = 1 << 16
    while True:
        buf = ctypes.create_string_buffer(cap)
        st = _ref_gguf.ref_gguf_dump(os.fsencode(path), buf, cap)
        if st != -2:
            return st, buf.value.decode(errors="replace")
        cap *= 4


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        L = ctypes.CDLL(os.path.join(HERE, "_ref", "libref_moe.so"))
        vp, i, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
        L.ref_dot_f32_f64.argtypes = [vp, vp, i]
        L.ref_dot_f32_f64.restype = ctypes.c_double
        L.ref_dot_f32_f64_portable.argtypes = [vp, vp, i]
        L.ref_dot_f32_f64_portable.restype = ctypes.c_double
        L.ref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.ref_fp16_to_fp32.restype = ctypes.c_float
        L.ref_dequant_q8_0.argtypes = [vp, i64, vp]
        L.ref_dequant_q4_k.argtypes = [vp, i64, vp]
        L.ref_moe_ffn_f32.argtypes = [vp, i, i, i, i, i, vp, vp, vp, vp, vp, i]
        L.ref_moe_ffn_f32_omp.argtypes = [vp, i, i, i, i, i, vp, vp, vp, vp, vp, i, i]
        L.ref_moe_ffn_routed_f32.argtypes = [vp, i, i, i, i, i, vp, vp, vp, vp, vp, i, i, vp, i, i]
        L.ref_matmul_f32_batch.argtypes = [vp, vp, vp, i, i, i]
        L.ref_silu.argtypes = [vp, vp, i64]
        L.ref_sigmoid.argtypes = [vp, vp, i64]
        L.ref_mul_col.argtypes = [vp, vp, vp, i, i]
        _ref = L
    return _ref


# ---- oracle wrappers (numpy in, numpy out) ----


def dot(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return ora().oracle_dot_f32_f64(a.ctypes.data, b.ctypes.data, a.size)


def dequant(type_id: int, raw: np.ndarray, n: int, first: int = 0) -> np.ndarray:
    raw = np.ascontiguousarray(raw)
    out = np.empty(n, np.float32)
    s = ora().oracle_dequant(type_id, raw.ctypes.data, first, n, out.ctypes.data)
    if s:
        raise ValueError(f"oracle_dequant status {s}")
    return out


def router_logits(x: np.ndarray, R: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    R = np.ascontiguousarray(R, np.float32)
    T, d = x.shape
    E = R.size // d
    out = np.empty((T, E), np.float32)
    ora().oracle_router_logits(x.ctypes.data, T, d, E, R.ctypes.data, out.ctypes.data)
    return out


def route(logits: np.ndarray, k: int, renorm=True, sigmoid=False, bias=None, groups_n=1, groups_top=1):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    idx = np.empty((T, k), np.int32)
    gates = np.empty((T, k), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    ora().oracle_route(logits.ctypes.data, T, E, k, int(renorm), int(sigmoid), _vp(b), groups_n, groups_top,
                       idx.ctypes.data, gates.ctypes.data)
    return idx, gates


def dispatch(idx: np.ndarray, E: int):
    idx = np.ascontiguousarray(idx, np.int32)
    T, k = idx.shape
    offsets = np.empty(E + 1, np.int32)
    perm = np.full(T * k, -1, np.int32)
    ora().oracle_dispatch(idx.ctypes.data, T, k, E, offsets.ctypes.data, perm.ctypes.data)
    return offsets, perm


def moe_layer(x, router, G, U, D, d_ff, E, k, renorm=True, sigmoid=False, bias=None, groups_n=1, groups_top=1,
              scale=1.0, d_ff_sh=0, Gs=None, Us=None, Ds=None, Wsg=None, sgate_out=None, nthreads=0) -> np.ndarray:
    """The whole layer on F32 stacks (moe_ffn_f32_cpu / moe_ffn_routed_f32_cpu + the IR's scale and
    shared expert; Wsg [d]: qwen2moe's shared-expert gate ffn_gate_inp_shexp), token-parallel over
    `nthreads` OpenMP threads (0: OpenMP's default). sgate_out [T], if given, receives the gate logits."""
    arrs = [np.ascontiguousarray(a, np.float32) if a is not None else None
            for a in (x, router, G, U, D, bias, Gs, Us, Ds, Wsg)]
    x, router, G, U, D, bias, Gs, Us, Ds, Wsg = arrs
    T, d = x.shape
    out = np.empty((T, d), np.float32)
    ora().oracle_moe_layer_gated(x.ctypes.data, T, d, d_ff, E, k, int(renorm), int(sigmoid), _vp(bias), groups_n,
                                 groups_top, float(scale), router.ctypes.data, G.ctypes.data, U.ctypes.data,
                                 D.ctypes.data, d_ff_sh, _vp(Gs), _vp(Us), _vp(Ds), _vp(Wsg), _vp(sgate_out),
                                 out.ctypes.data, nthreads)
    return out
