"""This project's GGUF reader (csrc/gguf.cpp, include/ember_gguf.h) against the reference's own reader
(load_gguf_meta, gguf_parser.cpp), compiled in place into oracle/_ref/libref_gguf.so.

On files written by ember_moe/gguf_writer.py (Mixtral-, DeepSeek- and qwen2moe-shaped layers, every
expert encoding, alignments 32 and 64, GGUF v2 and v3, scalar metadata of every width) both readers
must report the same tensors in the same order — name, ggml type, dimensions, offset and byte size —
and the same scalar metadata; on malformed files, every file the reference rejects must be rejected
here too (this reader also checks tensor extents against the file, which the reference's metadata pass
leaves to its data pass)."""
import os
import struct

import numpy as np
import pytest

import ember_moe as em
from ember_moe import gguf_writer as gw
from oracle import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_gguf_available(), reason="oracle/_ref/libref_gguf.so not built "
                                "(the reference sources are absent)")


@pytest.fixture(autouse=True)
def _log_in_tmp(tmp_path, monkeypatch):
    """The reference's logger (logger.cpp) appends to debugging.log in the working directory."""
    monkeypatch.chdir(tmp_path)


def _ours(path):
    with em.Gguf(path) as g:
        ts = []
        for t in g.tensors():
            ts.append((t.name.decode(), t.type, t.n_dims, tuple(t.ne[i] for i in range(t.n_dims)), t.offset, t.bytes))
        return g, ts


def _ref(path):
    st, text = O.ref_gguf_dump(path)
    assert st == 0, text
    head, meta, strings, tensors = None, {}, {}, []
    for ln in text.splitlines():
        kind, rest = ln[0], ln[2:]
        if kind == "H":
            head = tuple(int(v) for v in rest.split())
        elif kind == "M":
            k, v = rest.rsplit(" ", 1)
            meta[k] = float(v)
        elif kind == "S":
            k, _, v = rest.partition(" ")
            strings[k] = v
        elif kind == "T":
            f = rest.split()
            n = int(f[2])
            tensors.append((f[0], int(f[1]), n, tuple(int(v) for v in f[3:3 + n]), int(f[3 + n]), int(f[4 + n])))
    return head, meta, strings, tensors


def _compare(path, version):
    head, meta, strings, ref_t = _ref(path)
    with em.Gguf(path) as g:
        ours = [(t.name.decode(), t.type, t.n_dims, tuple(int(t.ne[i]) for i in range(t.n_dims)), int(t.offset),
                 int(t.bytes)) for t in g.tensors()]
        assert head[0] == version == g.version
        assert head[1] == len(ours)
        assert ours == ref_t
        for k, v in meta.items():
            assert g.number(k) == v, k
        for k, v in strings.items():
            assert g.string(k) == v, k
    return ref_t


LAYERS = {
    "mixtral-q8": ("llama", dict(d=256, d_ff=512, E=8, k=2, wtype=em.Q8_0)),
    "mixtral-q4k": ("llama", dict(d=256, d_ff=512, E=4, k=2, wtype=em.Q4_K)),
    "deepseek-bf16": ("deepseek2", dict(d=128, d_ff=192, E=16, k=4, wtype=em.BF16, scoring=em.SCORE_SIGMOID,
                                        bias_std=1.0, groups_n=4, groups_top=2, out_scale=2.5, d_ff_shared=256)),
    "qwen2moe-f16": ("qwen2moe", dict(d=128, d_ff=96, E=8, k=4, wtype=em.F16, renorm=False, d_ff_shared=128,
                                      shared_gated=True)),
    "qwen3moe-f32": ("qwen3moe", dict(d=64, d_ff=96, E=8, k=2, wtype=em.F32)),
}


@pytest.mark.parametrize("name", sorted(LAYERS))
@pytest.mark.parametrize("version,alignment", [(3, 32), (3, 64), (2, 32)])
def test_reader_matches_reference(tmp_path, name, version, alignment):
    arch, kw = LAYERS[name]
    hl = em.make_host_layer(em.LayerSpec(seed=4, **kw))
    other = em.make_host_layer(em.LayerSpec(seed=5, **kw))
    extra = {"general.name": "synthetic", f"{arch}.context_length": gw.Typed(gw.KV_U64, 4096),
             f"{arch}.rope.freq_base": gw.Typed(gw.KV_F64, 1e6), f"{arch}.attention.layer_norm_rms_epsilon": 1e-5,
             "general.file_type": gw.Typed(gw.KV_U16, 7), "general.quantized": True,
             f"{arch}.attention.head_count": gw.Typed(gw.KV_I8, 8)}
    p = str(tmp_path / f"{name}.gguf")
    gw.write_gguf(p, gw.moe_meta(arch, hl, 2, extra), gw.moe_layer_tensors(other, 0) + gw.moe_layer_tensors(hl, 1),
                  alignment=alignment, version=version)
    ref_t = _compare(p, version)
    assert len(ref_t) >= 8


def test_malformed_files(tmp_path):
    hl = em.make_host_layer(em.LayerSpec(d=64, d_ff=96, E=4, k=2, wtype=em.Q8_0, seed=3))
    t = gw.moe_layer_tensors(hl, 0)
    good_p = str(tmp_path / "good.gguf")
    gw.write_gguf(good_p, gw.moe_meta("llama", hl, 1), t)
    good = open(good_p, "rb").read()
    cases = {"magic": b"XGUF" + good[4:], "version 7": good[:4] + struct.pack("<I", 7) + good[8:],
             "empty": b"", "tensor count": good[:8] + struct.pack("<Q", 1 << 40) + good[16:]}
    for cut in (10, 30, 200, 700):
        cases[f"cut {cut}"] = good[:cut]
    rejected_by_ref = 0
    for what, blob in cases.items():
        p = str(tmp_path / f"bad_{len(blob)}_{abs(hash(what)) % 1000}.gguf")
        open(p, "wb").write(blob)
        st, msg = O.ref_gguf_dump(p)
        with pytest.raises(em.EmberError) as e:
            em.Gguf(p)
        assert e.value.status == em.ERR_FORMAT, what
        rejected_by_ref += st != 0
    assert rejected_by_ref >= 6  # the reference rejects the broken headers too
