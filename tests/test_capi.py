"""CPU checks of the C ABI library: it loads, exports every function include/*.h declares, and its
validation paths (which return before any GPU work) give the documented status codes."""
import ctypes
import os
import re

import numpy as np
import pytest

import ember_moe as em

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header: str):
    with open(os.path.join(ROOT, "include", header)) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(ember_\w+)\s*\(", text, flags=re.M)))


def exported(path: str):
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


def test_hip_library_exports_every_declared_symbol():
    names = declared("ember_moe.h")
    assert {"ember_moe_ffn", "ember_moe_scratch_bytes", "ember_moe_route", "ember_moe_router_logits",
            "ember_moe_ffn_timed", "ember_moe_route_scratch_bytes", "ember_moe_strerror"} <= set(names)
    missing = set(names) - exported(em.lib_path())
    assert not missing, missing
    em.lib()  # loads


def test_host_library_exports_every_declared_symbol():
    names = declared("ember_moe_host.h")
    assert "ember_quantize" in names and "ember_fill_normal" in names
    missing = set(names) - exported(em.host_lib_path())
    assert not missing, missing


def test_gguf_reader_exports_every_declared_symbol():
    names = declared("ember_gguf.h")
    assert {"ember_gguf_open", "ember_gguf_moe_layer", "ember_gguf_find_tensor"} <= set(names)
    missing = set(names) - exported(em.host_lib_path())
    assert not missing, missing
    assert {"ember_gguf_layer_bytes", "ember_gguf_upload_layer"} <= exported(em.lib_path())


def _layer(**kw):
    L = em.Layer()
    base = dict(d=256, d_ff=512, E=8, k=2, renorm=1, scoring=0, groups_n=1, groups_top=1, out_scale=1.0,
                router=0x1000, gate=0x2000, gate_type=em.Q8_0, up=0x3000, up_type=em.Q8_0, down=0x4000,
                down_type=em.Q8_0)
    base.update(kw)
    for k, v in base.items():
        setattr(L, k, v)
    return L


def test_scratch_bytes_and_validation():
    L = _layer()
    n1, n64 = em.scratch_bytes(L, 1), em.scratch_bytes(L, 64)
    assert 0 < n1 < n64
    assert em.scratch_bytes(_layer(E=0), 1) == 0
    assert em.scratch_bytes(_layer(k=65), 1) == 0
    assert em.scratch_bytes(_layer(gate_type=99), 1) == 0
    assert em.scratch_bytes(_layer(d=96), 1) == 0          # Q8_0 rows must be whole 64-element chunks
    assert em.scratch_bytes(_layer(gate=0x2004), 1) == 0   # 16-byte alignment
    assert em.scratch_bytes(_layer(groups_n=3), 1) == 0     # E % groups
    assert em.scratch_bytes(_layer(groups_n=4, groups_top=2), 1) > 0


@pytest.mark.parametrize("kw,status", [
    (dict(E=0), em.ERR_SHAPE), (dict(gate_type=3), em.ERR_TYPE), (dict(router=0), em.ERR_NULL),
    (dict(down=0x4008), em.ERR_ALIGN), (dict(up_type=em.BF16), em.ERR_TYPE),
])
def test_ffn_rejects_bad_descriptors_without_launching(kw, status):
    L = _layer(**kw)
    lib = em.lib()
    s = lib.ember_moe_ffn(ctypes.byref(L), 0x10000, 4, 0x20000, 0x30000, 1 << 30, None)
    assert s == status, em.strerror(s)


def test_ffn_rejects_small_scratch_and_null_io():
    L = _layer()
    lib = em.lib()
    need = em.scratch_bytes(L, 4)
    assert lib.ember_moe_ffn(ctypes.byref(L), 0x10000, 4, 0x20000, 0x30000, need - 1, None) == em.ERR_SCRATCH
    assert lib.ember_moe_ffn(ctypes.byref(L), 0, 4, 0x20000, 0x30000, need, None) == em.ERR_NULL
    assert lib.ember_moe_ffn(ctypes.byref(L), 0x10000, -1, 0x20000, 0x30000, need, None) == em.ERR_SHAPE
    assert lib.ember_moe_ffn(ctypes.byref(L), 0, 0, 0, 0, 0, None) == em.OK  # T = 0: nothing to do


def test_strerror():
    for s in (em.OK, em.ERR_SHAPE, em.ERR_TYPE, em.ERR_SCRATCH, em.ERR_NULL, em.ERR_LAUNCH, em.ERR_ALIGN,
              em.ERR_FORMAT, em.ERR_NOT_FOUND):
        assert em.strerror(s) and em.strerror(s) != "unknown status"


def test_prefill_pack_sizes_and_validation():
    # the pack holds every 256-row x 64-column tile of 68-byte rows: gate/up tiles per 128 columns of
    # h, down tiles per 256 output rows (partial tiles counted whole)
    def expect(d, d_ff, E):
        return E * (-(-d_ff // 128) * (d // 64) + -(-d // 256) * (d_ff // 64)) * 256 * 68

    L = _layer(d=512, d_ff=704, E=4)
    assert em.prefill_pack_bytes(L) == expect(512, 704, 4)
    assert em.prefill_pack_bytes(_layer(d=4096, d_ff=14336, E=8)) == expect(4096, 14336, 8)
    # only all-Q8_0 / all-Q4_K layers with whole 64-column tiles and all-BF16 layers have a pack
    # all-BF16 layers: int16 row exponents of gate, up [E][d_ff] and down [E][d] and a per-expert maximum
    # [E], each section 256-byte aligned
    bf = dict(gate_type=em.BF16, up_type=em.BF16, down_type=em.BF16)
    al = lambda v: -(-v // 256) * 256
    routed = 2 * al(8 * 512 * 2) + al(8 * 256 * 2) + al(8 * 2)
    assert em.prefill_pack_bytes(_layer(d=256, d_ff=512, E=8, **bf)) == routed
    # ... and the shared expert's rows when its stacks are BF16 too
    sh = dict(d_ff_shared=384, gate_shared=0x5000, gate_shared_type=em.BF16, up_shared=0x6000,
              up_shared_type=em.BF16, down_shared=0x7000, down_shared_type=em.BF16)
    assert em.prefill_pack_bytes(_layer(d=256, d_ff=512, E=8, **bf, **sh)) == (
        routed + 2 * al(384 * 2) + al(256 * 2) + al(2))
    assert em.prefill_pack_bytes(_layer(down_type=em.BF16)) == 0
    assert em.prefill_pack_bytes(_layer(d=512, d_ff=736)) == 0  # d_ff not a multiple of 64
    # all-Q4_K layers: 40-byte rows (the two groups' fp16 factors and the quarter's nibbles)
    q4 = dict(gate_type=em.Q4_K, up_type=em.Q4_K, down_type=em.Q4_K)
    assert em.prefill_pack_bytes(_layer(d=512, d_ff=768, E=4, **q4)) == expect(512, 768, 4) * 40 // 68
    assert em.prefill_pack_bytes(_layer(d=512, d_ff=768, E=4, gate_type=em.Q4_K, up_type=em.Q4_K)) == 0
    lib = em.lib()
    assert lib.ember_moe_prefill_pack(ctypes.byref(_layer(down_type=em.BF16)), 0x100000, 1 << 30, None) == em.ERR_TYPE
    assert lib.ember_moe_prefill_pack(ctypes.byref(L), 0, 1 << 30, None) == em.ERR_NULL
    assert lib.ember_moe_prefill_pack(ctypes.byref(L), 0x100080, 1 << 30, None) == em.ERR_ALIGN
    assert lib.ember_moe_prefill_pack(ctypes.byref(L), 0x100000, expect(512, 704, 4) - 1, None) == em.ERR_SCRATCH
    # a descriptor carrying a pack must be packable and the pack 256-byte aligned
    assert em.scratch_bytes(_layer(prefill_pack=0x100000), 1) > 0
    assert em.scratch_bytes(_layer(prefill_pack=0x100010), 1) == 0
    assert em.scratch_bytes(_layer(prefill_pack=0x100000, down_type=em.BF16), 1) == 0


@pytest.mark.parametrize("E,k,T", [(8, 2, 1), (8, 2, 9), (128, 8, 1), (64, 6, 4)])
def test_scratch_routing_view_layout(E, k, T):
    """ember_moe_scratch_routing (host arithmetic only): every section of the routing record lies inside
    the scratch, 4-byte aligned and disjoint from the others; the two u64 counters are adjacent words at
    the start of the flag area, whose 2E + 3 words (the counters, then one-token routing's exact and fast
    logit words, then the per-call conflict word) end before the logits."""
    L = _layer(E=E, k=k, d=512, d_ff=512)
    need = em.scratch_bytes(L, T)
    assert need > 0
    v = em.RoutingView()
    assert em.lib().ember_moe_scratch_routing(ctypes.byref(L), T, ctypes.byref(v)) == 0
    assert v.mismatches == v.fallbacks + 8 and v.fallbacks % 8 == 0
    assert v.conflict == v.fallbacks + 8 * (2 * E + 2)
    assert v.fallbacks + 8 * (2 * E + 3) <= v.logits
    spans = [(v.fallbacks, 8 * (2 * E + 3)), (v.logits, 4 * T * E), (v.idx, 4 * T * k), (v.gates, 4 * T * k),
             (v.offsets, 4 * (E + 1)), (v.perm, 4 * T * k), (v.pos, 4 * T * k), (v.used, 4 * E), (v.n_used, 4)]
    for off, n in spans:
        assert off % 4 == 0 and off + n <= need, (off, n, need)
    spans.sort()
    for (o1, n1), (o2, _) in zip(spans, spans[1:]):
        assert o1 + n1 <= o2, (o1, n1, o2)
