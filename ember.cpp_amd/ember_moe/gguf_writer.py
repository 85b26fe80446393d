"""GGUF writer (v3, little-endian) for MoE layers in llama.cpp's tensor layout.

The counterpart of the reader in include/ember_gguf.h: it lays out what the reference's loader reads
(gguf_parser.cpp; tensor names of weight_management.cpp:1162-1176 and graph_ir.cpp:640-660, 911-928)
— the header, typed metadata, tensor infos (name, dims in ggml ne order, type, offset) and the data
section aligned to general.alignment. Used to package synthetic layers (tests, benchmarks); real model
files come from llama.cpp's converters.
"""
from __future__ import annotations

import struct
from typing import Optional, Sequence

import numpy as np

KV_U8, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL = 0, 1, 2, 3, 4, 5, 6, 7
KV_STRING, KV_ARRAY, KV_U64, KV_I64, KV_F64 = 8, 9, 10, 11, 12

_SCALAR = {KV_U8: "<B", KV_I8: "<b", KV_U16: "<H", KV_I16: "<h", KV_U32: "<I", KV_I32: "<i", KV_F32: "<f",
           KV_BOOL: "<B", KV_U64: "<Q", KV_I64: "<q", KV_F64: "<d"}


class Typed:
    """A metadata value with an explicit GGUF type (e.g. Typed(KV_U64, n)); plain values are typed
    by _infer."""

    def __init__(self, kv_type: int, value):
        self.kv_type, self.value = kv_type, value


def _infer(v):
    if isinstance(v, bool):
        return KV_BOOL
    if isinstance(v, int):
        return KV_U32 if 0 <= v < 2**32 else KV_I64
    if isinstance(v, float):
        return KV_F32
    if isinstance(v, str):
        return KV_STRING
    if isinstance(v, (list, tuple)):
        return KV_ARRAY
    raise TypeError(f"no GGUF type for {type(v)}")


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == KV_STRING:
        return _string(v)
    if t == KV_ARRAY:
        et = _infer(v[0]) if len(v) else KV_U32
        return struct.pack("<IQ", et, len(v)) + b"".join(_value(et, e) for e in v)
    return struct.pack(_SCALAR[t], int(v) if t not in (KV_F32, KV_F64) else v)


def write_gguf(path: str, meta: dict, tensors: Sequence[tuple], alignment: int = 32, version: int = 3) -> None:
    """meta: {key: value or Typed(kv_type, value)}; tensors: (name, ggml_type, ne (ggml order), raw)."""
    meta = dict(meta)
    if alignment != 32:
        meta.setdefault("general.alignment", Typed(KV_U32, alignment))
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(meta))
    kv = b""
    for key, val in meta.items():
        t, v = (val.kv_type, val.value) if isinstance(val, Typed) else (_infer(val), val)
        kv += _string(key) + struct.pack("<I", t) + _value(t, v)
    infos, blobs, off = b"", [], 0
    for name, ttype, ne, raw in tensors:
        raw = np.ascontiguousarray(raw).view(np.uint8).reshape(-1)
        infos += _string(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", int(n)) for n in ne)
        infos += struct.pack("<IQ", int(ttype), off)
        blobs.append((off, raw))
        off += (raw.size + alignment - 1) // alignment * alignment
    body = head + kv + infos
    pad = (-len(body)) % alignment
    with open(path, "wb") as f:
        f.write(body + b"\0" * pad)
        pos = 0
        for o, raw in blobs:
            f.write(b"\0" * (o - pos))
            f.write(raw.tobytes())
            pos = o + raw.size
        f.write(b"\0" * ((-pos) % alignment))


def moe_layer_tensors(hl, layer: int, router_type: int = 0) -> list:
    """GGUF tensors of one ember_moe.HostLayer as llama.cpp names and lays them out: router
    ffn_gate_inp [E][d] (ne {d, E}), ffn_{gate,up}_exps ne {d, d_ff, E}, ffn_down_exps ne {d_ff, d, E},
    and for a DeepSeek-style layer exp_probs_b.bias and ffn_{gate,up,down}_shexp (qwen2moe's gated shared
    expert adds ffn_gate_inp_shexp)."""
    from . import F32, quantize

    s = hl.spec
    B = f"blk.{layer}."
    router = hl.router if router_type == F32 else quantize(router_type, hl.router)
    out = [(B + "ffn_gate_inp.weight", router_type, (s.d, s.E), router),
           (B + "ffn_gate_exps.weight", s.wtype, (s.d, s.d_ff, s.E), hl.gate),
           (B + "ffn_up_exps.weight", s.wtype, (s.d, s.d_ff, s.E), hl.up),
           (B + "ffn_down_exps.weight", s.wtype, (s.d_ff, s.d, s.E), hl.down)]
    if hl.bias is not None:
        out.append((B + "exp_probs_b.bias", F32, (s.E,), hl.bias))
    if s.d_ff_shared > 0:
        st = s.shared_type if s.shared_type is not None else s.wtype
        out += [(B + "ffn_gate_shexp.weight", st, (s.d, s.d_ff_shared), hl.gate_sh),
                (B + "ffn_up_shexp.weight", st, (s.d, s.d_ff_shared), hl.up_sh),
                (B + "ffn_down_shexp.weight", st, (s.d_ff_shared, s.d), hl.down_sh)]
        if hl.shared_gate is not None:
            out.append((B + "ffn_gate_inp_shexp.weight", F32, (s.d,), hl.shared_gate))
    return out


def moe_meta(arch: str, hl, n_layers: int, extra: Optional[dict] = None) -> dict:
    """The metadata the reader needs for arch: block count, expert count, experts used, width, and for
    deepseek2 the router options of hl.spec (gating function, renorm, scale, groups)."""
    s = hl.spec
    m = {"general.architecture": arch, f"{arch}.block_count": n_layers, f"{arch}.embedding_length": s.d,
         f"{arch}.expert_count": s.E, f"{arch}.expert_used_count": s.k}
    if arch == "deepseek2":
        m[f"{arch}.expert_gating_func"] = 2 if s.scoring == 1 else 1
        m[f"{arch}.expert_weights_norm"] = bool(s.renorm)
        m[f"{arch}.expert_weights_scale"] = float(s.out_scale)
        if s.groups_n > 1:
            m[f"{arch}.expert_group_count"] = s.groups_n
            m[f"{arch}.expert_group_used_count"] = s.groups_top
    if extra:
        m.update(extra)
    return m
