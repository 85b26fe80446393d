"""Python binding of the MI355X MoE FFN C ABI (include/ember_moe.h) and host utilities.

The C ABI is the product boundary; this module is a thin ctypes layer used by the tests and the
benchmark. Device memory and streams come from PyTorch (plumbing only): tensors are passed to the
library as raw pointers. There is no fallback: if ``libember_moe.so`` is missing, importing
``ember_moe.lib()`` raises.

Reference interface mirrored: ``moe_ffn_cuda`` / ``moe_ffn_scratch_floats`` (cuda_kernels.h:668-693)
— same arguments (x, T, d, d_ff, E, k, renorm, router, gate/up/down stacks, scratch, out, stream),
generalised to quantized expert stacks and the IR's router options (graph_ir.cpp:2677-2710).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# ggml type ids (ggml_types.h:20-40)
F32, F16, Q8_0, Q4_K, BF16 = 0, 1, 8, 12, 30
TYPE_NAMES = {F32: "f32", F16: "f16", Q8_0: "q8_0", Q4_K: "q4_k", BF16: "bf16"}
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}

SCORE_SOFTMAX, SCORE_SIGMOID = 0, 1

OK, ERR_SHAPE, ERR_TYPE, ERR_SCRATCH, ERR_NULL, ERR_LAUNCH, ERR_ALIGN = 0, -1, -2, -3, -4, -5, -6
ERR_FORMAT, ERR_NOT_FOUND = -7, -8


class EmberError(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} ({status})" if what else f"{strerror(status)} ({status})")


class Layer(ctypes.Structure):
    """ember_moe_layer (include/ember_moe.h)."""

    _fields_ = [
        ("d", ctypes.c_int), ("d_ff", ctypes.c_int), ("E", ctypes.c_int), ("k", ctypes.c_int),
        ("renorm", ctypes.c_int), ("scoring", ctypes.c_int),
        ("selection_bias", ctypes.c_void_p),
        ("groups_n", ctypes.c_int), ("groups_top", ctypes.c_int),
        ("out_scale", ctypes.c_float),
        ("router", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("gate_type", ctypes.c_int),
        ("up", ctypes.c_void_p), ("up_type", ctypes.c_int),
        ("down", ctypes.c_void_p), ("down_type", ctypes.c_int),
        ("d_ff_shared", ctypes.c_int),
        ("gate_shared", ctypes.c_void_p), ("gate_shared_type", ctypes.c_int),
        ("up_shared", ctypes.c_void_p), ("up_shared_type", ctypes.c_int),
        ("down_shared", ctypes.c_void_p), ("down_shared_type", ctypes.c_int),
        ("prefill_pack", ctypes.c_void_p),
        ("shared_gate", ctypes.c_void_p),
    ]


class RoutingView(ctypes.Structure):
    """ember_moe_routing_view (include/ember_moe.h): byte offsets of a call's routing in its scratch."""

    _fields_ = [(n, ctypes.c_size_t) for n in
                ("logits", "idx", "gates", "offsets", "perm", "pos", "used", "n_used", "fallbacks",
                 "mismatches", "conflict")]


_lib = None
_host = None


class GgufTensor(ctypes.Structure):
    """ember_gguf_tensor (include/ember_gguf.h)."""

    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int), ("n_dims", ctypes.c_int),
                ("ne", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]


class GgufMoe(ctypes.Structure):
    """ember_gguf_moe (include/ember_gguf.h)."""

    _fields_ = [("layer", ctypes.c_int), ("d", ctypes.c_int), ("d_ff", ctypes.c_int), ("E", ctypes.c_int),
                ("k", ctypes.c_int), ("renorm", ctypes.c_int), ("scoring", ctypes.c_int),
                ("groups_n", ctypes.c_int), ("groups_top", ctypes.c_int), ("out_scale", ctypes.c_float),
                ("d_ff_shared", ctypes.c_int),
                ("router", GgufTensor), ("gate", GgufTensor), ("up", GgufTensor), ("down", GgufTensor),
                ("bias", GgufTensor), ("gate_shared", GgufTensor), ("up_shared", GgufTensor),
                ("down_shared", GgufTensor), ("shared_gate", GgufTensor)]


def lib_path() -> str:
    return os.path.join(_PKG_DIR, "libember_moe.so")


def host_lib_path() -> str:
    return os.path.join(_PKG_DIR, "libember_moe_host.so")


def lib() -> ctypes.CDLL:
    """The HIP library. Raises if it has not been built (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        p = lib_path()
        if not os.path.exists(p):
            raise RuntimeError(f"{p} is missing: build it with __graft_entry__.build() (no fallback path exists)")
        L = ctypes.CDLL(p)
        vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.ember_moe_scratch_bytes.argtypes = [ctypes.POINTER(Layer), i]
        L.ember_moe_scratch_bytes.restype = sz
        L.ember_moe_ffn.argtypes = [ctypes.POINTER(Layer), vp, i, vp, vp, sz, vp]
        L.ember_moe_ffn.restype = i
        L.ember_moe_ffn_noalloc.argtypes = [ctypes.POINTER(Layer), vp, i, vp, vp]
        L.ember_moe_ffn_noalloc.restype = i
        L.ember_moe_ffn_timed.argtypes = [ctypes.POINTER(Layer), vp, i, vp, vp, sz, vp, ctypes.POINTER(ctypes.c_float)]
        L.ember_moe_ffn_timed.restype = i
        L.ember_moe_router_logits.argtypes = [vp, i, i, i, vp, vp, vp]
        L.ember_moe_router_logits.restype = i
        L.ember_moe_route_scratch_bytes.argtypes = [i, i, i]
        L.ember_moe_route_scratch_bytes.restype = sz
        L.ember_moe_route.argtypes = [vp, i, i, i, i, i, vp, i, i, vp, vp, vp, vp, vp, sz, vp]
        L.ember_moe_route.restype = i
        L.ember_moe_prefill_pack_bytes.argtypes = [ctypes.POINTER(Layer)]
        L.ember_moe_prefill_pack_bytes.restype = sz
        L.ember_moe_prefill_pack.argtypes = [ctypes.POINTER(Layer), vp, sz, vp]
        L.ember_moe_prefill_pack.restype = i
        L.ember_moe_path.argtypes = [ctypes.POINTER(Layer), i]
        L.ember_moe_path.restype = i
        L.ember_moe_scratch_routing.argtypes = [ctypes.POINTER(Layer), i, ctypes.POINTER(RoutingView)]
        L.ember_moe_scratch_routing.restype = i
        L.ember_moe_strerror.argtypes = [i]
        L.ember_moe_strerror.restype = ctypes.c_char_p
        L.ember_gguf_layer_bytes.argtypes = [ctypes.POINTER(GgufMoe)]
        L.ember_gguf_layer_bytes.restype = sz
        L.ember_gguf_upload_layer.argtypes = [ctypes.POINTER(GgufMoe), vp, sz, ctypes.POINTER(Layer), vp]
        L.ember_gguf_upload_layer.restype = i
        _lib = L
    return _lib


def host() -> ctypes.CDLL:
    global _host
    if _host is None:
        p = host_lib_path()
        if not os.path.exists(p):
            raise RuntimeError(f"{p} is missing: build it with __graft_entry__.build()")
        H = ctypes.CDLL(p)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        H.ember_fill_normal.argtypes = [vp, i64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float]
        H.ember_fill_normal.restype = None
        H.ember_row_bytes.argtypes = [ctypes.c_int, i64]
        H.ember_row_bytes.restype = i64
        H.ember_quantize.argtypes = [ctypes.c_int, vp, i64, vp]
        H.ember_quantize.restype = ctypes.c_int
        H.ember_dequantize.argtypes = [ctypes.c_int, vp, i64, vp]
        H.ember_dequantize.restype = ctypes.c_int
        H.ember_f32_to_f16.argtypes = [ctypes.c_float]
        H.ember_f32_to_f16.restype = ctypes.c_uint16
        H.ember_f16_to_f32.argtypes = [ctypes.c_uint16]
        H.ember_f16_to_f32.restype = ctypes.c_float
        H.ember_f32_to_bf16.argtypes = [ctypes.c_float]
        H.ember_f32_to_bf16.restype = ctypes.c_uint16
        pp = ctypes.POINTER(ctypes.c_void_p)
        H.ember_gguf_open.argtypes = [ctypes.c_char_p, pp]
        H.ember_gguf_open.restype = ctypes.c_int
        H.ember_gguf_close.argtypes = [vp]
        H.ember_gguf_close.restype = None
        H.ember_gguf_version.argtypes = [vp]
        H.ember_gguf_version.restype = ctypes.c_int
        H.ember_gguf_n_tensors.argtypes = [vp]
        H.ember_gguf_n_tensors.restype = i64
        H.ember_gguf_tensor_at.argtypes = [vp, i64, ctypes.POINTER(GgufTensor)]
        H.ember_gguf_tensor_at.restype = ctypes.c_int
        H.ember_gguf_find_tensor.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]
        H.ember_gguf_find_tensor.restype = ctypes.c_int
        H.ember_gguf_meta_number.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]
        H.ember_gguf_meta_number.restype = ctypes.c_int
        H.ember_gguf_meta_string.argtypes = [vp, ctypes.c_char_p]
        H.ember_gguf_meta_string.restype = ctypes.c_char_p
        H.ember_gguf_arch.argtypes = [vp]
        H.ember_gguf_arch.restype = ctypes.c_char_p
        H.ember_gguf_n_layers.argtypes = [vp]
        H.ember_gguf_n_layers.restype = ctypes.c_int
        H.ember_gguf_moe_layer.argtypes = [vp, ctypes.c_int, ctypes.POINTER(GgufMoe)]
        H.ember_gguf_moe_layer.restype = ctypes.c_int
        H.ember_ggml_nbytes.argtypes = [ctypes.c_int, i64]
        H.ember_ggml_nbytes.restype = i64
        _host = H
    return _host


def strerror(status: int) -> str:
    try:
        return lib().ember_moe_strerror(status).decode()
    except RuntimeError:
        return f"status {status}"


def _ptr(a) -> int:
    if a is None:
        return 0
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()  # torch tensor


# ----------------------------------------------------------------------------------------------
# Host data utilities


def normal(n: int, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    host().ember_fill_normal(out.ctypes.data, n, seed, stream, mean, std)
    return out


def row_bytes(type_id: int, n: int) -> int:
    return int(host().ember_row_bytes(type_id, n))


def quantize(type_id: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    nbytes = row_bytes(type_id, x.size)
    if nbytes < 0:
        raise EmberError(ERR_SHAPE, f"quantize {TYPE_NAMES.get(type_id, type_id)} of {x.size} elements")
    out = np.empty(nbytes, dtype=np.uint8)
    s = host().ember_quantize(type_id, x.ctypes.data, x.size, out.ctypes.data)
    if s:
        raise EmberError(s, "quantize")
    return out


def dequantize(type_id: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw)
    out = np.empty(n, dtype=np.float32)
    s = host().ember_dequantize(type_id, raw.ctypes.data, n, out.ctypes.data)
    if s:
        raise EmberError(s, "dequantize")
    return out


# ----------------------------------------------------------------------------------------------
# Device entry points (torch tensors on the GPU; stream defaults to torch's current stream)


def _stream(stream) -> int:
    if stream is not None:
        return int(stream)
    import torch

    return int(torch.cuda.current_stream().cuda_stream)


def scratch_bytes(layer: Layer, T: int) -> int:
    return int(lib().ember_moe_scratch_bytes(ctypes.byref(layer), T))


def prefill_pack_bytes(layer: Layer) -> int:
    """Bytes of the layer's prefill pack (0: the layer has none — not all-Q8_0, all-Q4_K or all-BF16, or an
    invalid descriptor)."""
    return int(lib().ember_moe_prefill_pack_bytes(ctypes.byref(layer)))


def prefill_pack(layer: Layer, pack, stream=None) -> None:
    """Fills `pack` (a device tensor of prefill_pack_bytes(layer) bytes) and points layer.prefill_pack
    at it. Raises EmberError on failure."""
    n = pack.numel() * pack.element_size()
    st = int(lib().ember_moe_prefill_pack(ctypes.byref(layer), _ptr(pack), n, _stream(stream)))
    if st:
        raise EmberError(st, "ember_moe_prefill_pack")
    layer.prefill_pack = _ptr(pack)


def moe_ffn(layer: Layer, x, T: int, out, scratch, scratch_nbytes: Optional[int] = None, stream=None) -> int:
    """Calls ember_moe_ffn; returns the status (0 on success)."""
    n = scratch_nbytes if scratch_nbytes is not None else (scratch.numel() * scratch.element_size() if scratch is not None else 0)
    return int(lib().ember_moe_ffn(ctypes.byref(layer), _ptr(x), T, _ptr(out), _ptr(scratch), n, _stream(stream)))


# ember_moe_path bits (include/ember_moe.h)
PATH_GEMV, PATH_TILES64, PATH_TILES256 = 1, 2, 4
PATH_FUSED_ROUTE, PATH_SLICES, PATH_DOWN1, PATH_SHARED_MFMA = 8, 16, 32, 64


def path(layer: Layer, T: int) -> int:
    """The EMBER_PATH_* bits of the kernels a call with T tokens runs (ember_moe_path)."""
    st = lib().ember_moe_path(ctypes.byref(layer), T)
    if st < 0:
        raise EmberError(st, "ember_moe_path")
    return st


def scratch_routing(layer: Layer, T: int, scratch) -> dict:
    """The routing a completed ember_moe_ffn call left in `scratch` (a uint8 device tensor), copied to the
    host: logits [T][E], idx / gates [T][k], offsets [E+1], perm / pos [T*k], used [n_used], fallbacks, mismatches, conflict."""
    v = RoutingView()
    st = lib().ember_moe_scratch_routing(ctypes.byref(layer), T, ctypes.byref(v))
    if st:
        raise EmberError(st, "ember_moe_scratch_routing")
    E, k = layer.E, layer.k
    raw = scratch.cpu().numpy()

    def arr(off, n, dt):
        return raw[off:off + n * np.dtype(dt).itemsize].view(dt).copy()

    n_used = int(arr(v.n_used, 1, np.int32)[0])
    return dict(logits=arr(v.logits, T * E, np.float32).reshape(T, E),
                idx=arr(v.idx, T * k, np.int32).reshape(T, k), gates=arr(v.gates, T * k, np.float32).reshape(T, k),
                offsets=arr(v.offsets, E + 1, np.int32), perm=arr(v.perm, T * k, np.int32),
                pos=arr(v.pos, T * k, np.int32), used=arr(v.used, max(min(n_used, E), 0), np.int32),
                n_used=n_used, fallbacks=int(arr(v.fallbacks, 1, np.uint64)[0]),
                mismatches=int(arr(v.mismatches, 1, np.uint64)[0]),
                conflict=int(arr(v.conflict, 1, np.uint64)[0]))


NOALLOC_SCRATCH_BYTES = 32 << 20  # EMBER_MOE_NOALLOC_SCRATCH_BYTES


def moe_ffn_noalloc(layer: Layer, x, T: int, out, stream=None) -> int:
    """Calls ember_moe_ffn_noalloc (the library's own static scratch); returns the status."""
    return int(lib().ember_moe_ffn_noalloc(ctypes.byref(layer), _ptr(x), T, _ptr(out), _stream(stream)))


PHASES = ("router", "route", "dispatch", "gate_up", "down", "shared", "combine")


def moe_ffn_timed(layer: Layer, x, T: int, out, scratch, stream=None):
    """ember_moe_ffn_timed: runs the layer once, returns {phase: milliseconds}."""
    ms = (ctypes.c_float * len(PHASES))()
    n = scratch.numel() * scratch.element_size()
    s = int(lib().ember_moe_ffn_timed(ctypes.byref(layer), _ptr(x), T, _ptr(out), _ptr(scratch), n, _stream(stream), ms))
    if s:
        raise EmberError(s, "ember_moe_ffn_timed")
    return dict(zip(PHASES, list(ms)))


def router_logits(x, T: int, d: int, E: int, router, logits, stream=None) -> int:
    return int(lib().ember_moe_router_logits(_ptr(x), T, d, E, _ptr(router), _ptr(logits), _stream(stream)))


def route_scratch_bytes(T: int, E: int, k: int) -> int:
    return int(lib().ember_moe_route_scratch_bytes(T, E, k))


def route(logits, T, E, k, renorm, scoring, bias, groups_n, groups_top, idx, gates, offsets, perm, scratch,
          stream=None) -> int:
    n = scratch.numel() * scratch.element_size()
    return int(lib().ember_moe_route(_ptr(logits), T, E, k, int(renorm), scoring, _ptr(bias), groups_n, groups_top,
                                     _ptr(idx), _ptr(gates), _ptr(offsets), _ptr(perm), _ptr(scratch), n,
                                     _stream(stream)))


# ----------------------------------------------------------------------------------------------
# Synthetic layers: weights generated on the host by the seeded generator,
# quantized by this project's quantizers, uploaded once.


@dataclass
class LayerSpec:
    d: int
    d_ff: int
    E: int
    k: int
    wtype: int = F32
    renorm: bool = True
    scoring: int = SCORE_SOFTMAX
    bias_std: float = 0.0          # > 0: seeded selection bias ~ N(0, bias_std)
    groups_n: int = 1
    groups_top: int = 1
    out_scale: float = 1.0
    d_ff_shared: int = 0
    shared_type: Optional[int] = None
    shared_gated: bool = False     # qwen2moe: the shared expert scaled by sigmoid(shared_gate . x)
    weight_std: float = 0.02
    router_std: Optional[float] = None  # default 1/sqrt(d)
    seed: int = 0


# generator streams for each tensor of a layer
_STREAM = {"router": 1, "gate": 2, "up": 3, "down": 4, "bias": 5, "gate_sh": 6, "up_sh": 7, "down_sh": 8,
           "shared_gate": 9, "x": 100}


@dataclass
class HostLayer:
    """Host copies: encoded bytes per tensor (the GGUF payload) and the spec."""

    spec: LayerSpec
    router: np.ndarray
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    bias: Optional[np.ndarray] = None
    gate_sh: Optional[np.ndarray] = None
    up_sh: Optional[np.ndarray] = None
    down_sh: Optional[np.ndarray] = None
    shared_gate: Optional[np.ndarray] = None  # f32 [d] (qwen2moe's ffn_gate_inp_shexp)

    def dequantized(self, name: str) -> np.ndarray:
        """The F32 stack the reference would hold after dequantize-at-load (weight_management.cpp:802-877)."""
        s = self.spec
        raw = getattr(self, name)
        if name in ("gate", "up"):
            n, t = s.E * s.d_ff * s.d, s.wtype
        elif name == "down":
            n, t = s.E * s.d * s.d_ff, s.wtype
        else:
            n, t = s.d * s.d_ff_shared, (s.shared_type if s.shared_type is not None else s.wtype)
        return dequantize(t, raw, n)


def make_host_layer(spec: LayerSpec) -> HostLayer:
    s = spec
    rstd = s.router_std if s.router_std is not None else 1.0 / np.sqrt(s.d)
    router = normal(s.E * s.d, s.seed, _STREAM["router"], 0.0, rstd)

    def stack(name, n, t):
        return quantize(t, normal(n, s.seed, _STREAM[name], 0.0, s.weight_std))

    hl = HostLayer(spec=s, router=router,
                   gate=stack("gate", s.E * s.d_ff * s.d, s.wtype),
                   up=stack("up", s.E * s.d_ff * s.d, s.wtype),
                   down=stack("down", s.E * s.d * s.d_ff, s.wtype))
    if s.bias_std > 0:
        hl.bias = normal(s.E, s.seed, _STREAM["bias"], 0.0, s.bias_std)
    if s.d_ff_shared > 0:
        st = s.shared_type if s.shared_type is not None else s.wtype
        hl.gate_sh = stack("gate_sh", s.d_ff_shared * s.d, st)
        hl.up_sh = stack("up_sh", s.d_ff_shared * s.d, st)
        hl.down_sh = stack("down_sh", s.d * s.d_ff_shared, st)
        if s.shared_gated:
            hl.shared_gate = normal(s.d, s.seed, _STREAM["shared_gate"], 0.0, 1.0 / np.sqrt(s.d))
    return hl


def make_input(spec: LayerSpec, T: int, seed: Optional[int] = None) -> np.ndarray:
    return normal(T * spec.d, spec.seed if seed is None else seed, _STREAM["x"], 0.0, 1.0).reshape(T, spec.d)


@dataclass
class DeviceLayer:
    """Device-resident tensors of one layer and the C descriptor pointing at them."""

    host: HostLayer
    tensors: dict = field(default_factory=dict)
    desc: Layer = field(default_factory=Layer)

    @staticmethod
    def upload(hl: HostLayer, device="cuda") -> "DeviceLayer":
        import torch

        dl = DeviceLayer(host=hl)
        s = hl.spec

        def up(a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(device)

        for name in ("router", "gate", "up", "down", "bias", "gate_sh", "up_sh", "down_sh", "shared_gate"):
            a = getattr(hl, name)
            if a is not None:
                dl.tensors[name] = up(a)
        t = dl.tensors
        L = dl.desc
        L.d, L.d_ff, L.E, L.k = s.d, s.d_ff, s.E, s.k
        L.renorm, L.scoring = int(s.renorm), s.scoring
        L.selection_bias = _ptr(t.get("bias"))
        L.groups_n, L.groups_top = s.groups_n, s.groups_top
        L.out_scale = s.out_scale
        L.router = _ptr(t["router"])
        L.gate, L.gate_type = _ptr(t["gate"]), s.wtype
        L.up, L.up_type = _ptr(t["up"]), s.wtype
        L.down, L.down_type = _ptr(t["down"]), s.wtype
        L.d_ff_shared = s.d_ff_shared
        if s.d_ff_shared > 0:
            st = s.shared_type if s.shared_type is not None else s.wtype
            L.gate_shared, L.gate_shared_type = _ptr(t["gate_sh"]), st
            L.up_shared, L.up_shared_type = _ptr(t["up_sh"]), st
            L.down_shared, L.down_shared_type = _ptr(t["down_sh"]), st
            L.shared_gate = _ptr(t.get("shared_gate"))
        return dl

    def clone(self) -> "DeviceLayer":
        """A second device copy of the layer (every tensor, the prefill pack included) with its own
        descriptor: the same weights at other addresses, e.g. to time calls that do not find the previous
        call's weights in the device's last-level cache, as consecutive layers of a model do not."""
        c = DeviceLayer(host=self.host)
        ctypes.memmove(ctypes.byref(c.desc), ctypes.byref(self.desc), ctypes.sizeof(Layer))
        fields = {"router": "router", "gate": "gate", "up": "up", "down": "down", "bias": "selection_bias",
                  "gate_sh": "gate_shared", "up_sh": "up_shared", "down_sh": "down_shared",
                  "shared_gate": "shared_gate", "pack": "prefill_pack"}
        for name, t in self.tensors.items():
            c.tensors[name] = t.clone()
            if name in fields:
                setattr(c.desc, fields[name], _ptr(c.tensors[name]))
        return c

    def forward(self, x, out=None, scratch=None, stream=None):
        """Runs ember_moe_ffn on device tensor x [T][d]; returns (out, scratch)."""
        import torch

        T = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        need = scratch_bytes(self.desc, T)
        if need == 0:
            raise EmberError(ERR_SHAPE, "ember_moe_scratch_bytes")
        if scratch is None or scratch.numel() < need:
            scratch = torch.empty(need, dtype=torch.uint8, device=x.device)
        s = moe_ffn(self.desc, x, T, out, scratch, stream=stream)
        if s:
            raise EmberError(s, "ember_moe_ffn")
        return out, scratch


# ----------------------------------------------------------------------------------------------
# GGUF files (include/ember_gguf.h; the reader is in libember_moe_host.so, the upload in libember_moe.so)


class Gguf:
    """An open GGUF file (ember_gguf_open). The mapped tensor data stays valid until close()."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        st = host().ember_gguf_open(os.fsencode(path), ctypes.byref(h))
        if st != OK:
            raise EmberError(st, f"ember_gguf_open({path})")
        self._h = h

    def close(self):
        if self._h:
            host().ember_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def version(self) -> int:
        return host().ember_gguf_version(self._h)

    @property
    def arch(self) -> str:
        return host().ember_gguf_arch(self._h).decode()

    @property
    def n_layers(self) -> int:
        return host().ember_gguf_n_layers(self._h)

    def tensors(self):
        out = []
        for i in range(host().ember_gguf_n_tensors(self._h)):
            t = GgufTensor()
            st = host().ember_gguf_tensor_at(self._h, i, ctypes.byref(t))
            if st != OK:
                raise EmberError(st, "ember_gguf_tensor_at")
            out.append(t)
        return out

    def find(self, name: str) -> Optional[GgufTensor]:
        t = GgufTensor()
        st = host().ember_gguf_find_tensor(self._h, name.encode(), ctypes.byref(t))
        if st == ERR_NOT_FOUND:
            return None
        if st != OK:
            raise EmberError(st, "ember_gguf_find_tensor")
        return t

    def tensor_bytes(self, t: GgufTensor) -> np.ndarray:
        return np.ctypeslib.as_array(ctypes.cast(t.data, ctypes.POINTER(ctypes.c_uint8)), shape=(t.bytes,)).copy()

    def number(self, key: str) -> Optional[float]:
        v = ctypes.c_double()
        return v.value if host().ember_gguf_meta_number(self._h, key.encode(), ctypes.byref(v)) == OK else None

    def string(self, key: str) -> Optional[str]:
        r = host().ember_gguf_meta_string(self._h, key.encode())
        return None if r is None else r.decode()

    def moe_layer(self, layer: int) -> GgufMoe:
        m = GgufMoe()
        st = host().ember_gguf_moe_layer(self._h, layer, ctypes.byref(m))
        if st != OK:
            raise EmberError(st, f"ember_gguf_moe_layer({layer})")
        m._owner = self  # the view points into this file's mapping
        return m


def gguf_layer_bytes(m: GgufMoe) -> int:
    return lib().ember_gguf_layer_bytes(ctypes.byref(m))


def gguf_upload_layer(m: GgufMoe, dev, stream=None) -> Layer:
    """Uploads a GGUF MoE layer into `dev` (a uint8 device tensor of at least gguf_layer_bytes(m))."""
    L = Layer()
    st = lib().ember_gguf_upload_layer(ctypes.byref(m), _ptr(dev), dev.numel(), ctypes.byref(L), _stream(stream))
    if st != OK:
        raise EmberError(st, "ember_gguf_upload_layer")
    L._owner = dev
    return L
