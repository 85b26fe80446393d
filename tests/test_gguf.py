"""CPU tests of the GGUF reader (include/ember_gguf.h, libember_moe_host.so): files written by
ember_moe.gguf_writer are read back tensor by tensor, the MoE layer view follows the reference's IR
builder per architecture (graph_ir.cpp:681-705, 832-851, 911-928), and malformed files are rejected
with EMBER_ERR_FORMAT rather than read out of bounds."""
import os
import struct

import numpy as np
import pytest

import ember_moe as em
from ember_moe import gguf_writer as gw


def _layer(arch_opts=None, **kw):
    spec = dict(d=64, d_ff=96, E=4, k=2, wtype=em.Q8_0, seed=3)
    spec.update(kw)
    return em.make_host_layer(em.LayerSpec(**spec))


def _write(tmp_path, name, meta, tensors, **kw):
    p = os.path.join(tmp_path, name)
    gw.write_gguf(p, meta, tensors, **kw)
    return p


def test_llama_moe_file_reads_back(tmp_path):
    hl0, hl1 = _layer(), _layer(seed=4, wtype=em.BF16)
    extra = {"tokenizer.ggml.tokens": ["<s>", "</s>", "hello"], "llama.rope.freq_base": 1e6,
             "general.name": "synthetic", "llama.big": gw.Typed(gw.KV_U64, 2**40), "llama.neg": -5}
    tensors = [("token_embd.weight", em.F16, (64, 10), np.arange(640, dtype=np.uint16)),
               ("unknown_kind.weight", 16, (256,), np.zeros(66, np.uint8))]  # a type this reader does not size
    tensors += gw.moe_layer_tensors(hl0, 0) + gw.moe_layer_tensors(hl1, 1, router_type=em.BF16)
    p = _write(tmp_path, "m.gguf", gw.moe_meta("llama", hl0, 3, extra), tensors)
    with em.Gguf(p) as g:
        assert g.version == 3 and g.arch == "llama" and g.n_layers == 3
        ts = g.tensors()
        assert [t.name.decode() for t in ts] == [t[0] for t in tensors]
        for t, (name, ttype, ne, raw) in zip(ts, tensors):
            assert t.type == ttype and list(t.ne[: len(ne)]) == list(ne) and t.offset % 32 == 0
            if ttype != 16:
                assert np.array_equal(g.tensor_bytes(t), np.ascontiguousarray(raw).view(np.uint8).reshape(-1))
            else:
                assert t.bytes == 0
        assert g.number("llama.expert_count") == 4 and g.number("llama.big") == 2**40
        assert g.number("llama.neg") == -5 and g.number("llama.rope.freq_base") == pytest.approx(1e6)
        assert g.string("general.name") == "synthetic" and g.string("llama.expert_count") is None
        assert g.number("tokenizer.ggml.tokens") is None and g.find("nope") is None
        m = g.moe_layer(0)
        assert (m.d, m.d_ff, m.E, m.k, m.renorm, m.scoring) == (64, 96, 4, 2, 1, em.SCORE_SOFTMAX)
        assert (m.groups_n, m.out_scale, m.d_ff_shared) == (1, 1.0, 0) and m.bias.name is None
        assert m.gate.type == em.Q8_0 and m.down.ne[0] == 96 and m.down.ne[1] == 64
        m1 = g.moe_layer(1)
        assert m1.gate.type == em.BF16 and m1.router.type == em.BF16
        with pytest.raises(em.EmberError) as e:
            g.moe_layer(2)  # no tensors for block 2
        assert e.value.status == em.ERR_NOT_FOUND


def test_deepseek2_router_options_and_shared_expert(tmp_path):
    hl = _layer(E=8, k=3, scoring=em.SCORE_SIGMOID, renorm=True, bias_std=2.0, groups_n=4, groups_top=2,
                out_scale=2.5, d_ff_shared=64)
    p = _write(tmp_path, "ds.gguf", gw.moe_meta("deepseek2", hl, 2), gw.moe_layer_tensors(hl, 1))
    with em.Gguf(p) as g:
        with pytest.raises(em.EmberError) as e:
            g.moe_layer(0)  # a leading dense block: no MoE tensors
        assert e.value.status == em.ERR_NOT_FOUND
        m = g.moe_layer(1)
        assert (m.E, m.k, m.scoring, m.renorm, m.groups_n, m.groups_top) == (8, 3, em.SCORE_SIGMOID, 1, 4, 2)
        assert m.out_scale == 2.5 and m.d_ff_shared == 64 and m.bias.name.decode() == "blk.1.exp_probs_b.bias"
        assert np.array_equal(g.tensor_bytes(m.bias).view(np.float32), hl.bias)


@pytest.mark.parametrize("arch,renorm", [("qwen3moe", 1), ("qwen2moe", 0), ("mistral", 1)])
def test_qwen_and_mistral_gates(tmp_path, arch, renorm):
    hl = _layer()
    p = _write(tmp_path, f"{arch}.gguf", gw.moe_meta(arch, hl, 1), gw.moe_layer_tensors(hl, 0))
    with em.Gguf(p) as g:
        assert g.moe_layer(0).renorm == renorm


def test_qwen2moe_gated_shared_expert(tmp_path):
    """graph_ir.cpp:700-706: qwen2moe's shared expert counts only when ffn_gate_inp_shexp gates it."""
    hl = _layer(d_ff_shared=128, shared_gated=True)
    assert hl.shared_gate is not None
    t = gw.moe_layer_tensors(hl, 0)
    p = _write(tmp_path, "q2.gguf", gw.moe_meta("qwen2moe", hl, 1), t)
    with em.Gguf(p) as g:
        m = g.moe_layer(0)
        assert (m.renorm, m.d_ff_shared) == (0, 128)
        assert m.shared_gate.name.decode() == "blk.0.ffn_gate_inp_shexp.weight"
        assert np.array_equal(g.tensor_bytes(m.shared_gate).view(np.float32), hl.shared_gate)
    # the same shared expert without its gate: the reference's graph leaves it out
    ungated = [x for x in t if "gate_inp_shexp" not in x[0]]
    p = _write(tmp_path, "q2u.gguf", gw.moe_meta("qwen2moe", hl, 1), ungated)
    with em.Gguf(p) as g:
        m = g.moe_layer(0)
        assert m.d_ff_shared == 0 and not m.shared_gate.name


def test_unsupported_layers(tmp_path):
    hl = _layer()
    t = gw.moe_layer_tensors(hl, 0)
    gate_only = t + [("blk.0.ffn_gate_inp_shexp.weight", em.F32, (64,), np.zeros(64, np.float32))]
    cases = {
        "qwen2moe shared-expert gate without the shared expert": (gw.moe_meta("qwen2moe", hl, 1), gate_only),
        "unknown architecture": (gw.moe_meta("gpt2", hl, 1), t),
        "expert_count disagrees": (gw.moe_meta("llama", hl, 1, {"llama.expert_count": 5}), t),
        "expert_used_count > E": (gw.moe_meta("llama", hl, 1, {"llama.expert_used_count": 9}), t),
        "down shape": (gw.moe_meta("llama", hl, 1), t[:3] + [(t[3][0], t[3][1], (64, 96, 4), t[3][3])]),
        "deepseek gating 3": (gw.moe_meta("deepseek2", hl, 1, {"deepseek2.expert_gating_func": 3}), t),
    }
    for i, (what, (meta, tensors)) in enumerate(cases.items()):
        with em.Gguf(_write(tmp_path, f"u{i}.gguf", meta, tensors)) as g:
            with pytest.raises(em.EmberError) as e:
                g.moe_layer(0)
            assert e.value.status == em.ERR_SHAPE, what


def _valid_bytes(tmp_path):
    hl = _layer()
    p = _write(tmp_path, "v.gguf", gw.moe_meta("llama", hl, 1), gw.moe_layer_tensors(hl, 0))
    return bytearray(open(p, "rb").read())


def _expect_format_error(tmp_path, blob, name):
    p = os.path.join(tmp_path, name)
    open(p, "wb").write(bytes(blob))
    with pytest.raises(em.EmberError) as e:
        em.Gguf(p)
    assert e.value.status == em.ERR_FORMAT, name


def test_malformed_files_are_rejected(tmp_path):
    good = _valid_bytes(tmp_path)
    with em.Gguf(os.path.join(tmp_path, "v.gguf")):
        pass
    bad_magic = bytearray(good)
    bad_magic[0] = ord("X")
    _expect_format_error(tmp_path, bad_magic, "magic.gguf")
    bad_version = bytearray(good)
    bad_version[4:8] = struct.pack("<I", 7)
    _expect_format_error(tmp_path, bad_version, "version.gguf")
    for cut in (10, 30, 200, 700, len(good) - 100):  # inside the header, metadata, tensor infos and data
        _expect_format_error(tmp_path, good[:cut], f"cut{cut}.gguf")
    huge = bytearray(good)
    huge[8:16] = struct.pack("<Q", 1 << 40)  # tensor count
    _expect_format_error(tmp_path, huge, "count.gguf")
    _expect_format_error(tmp_path, b"", "empty.gguf")
    with pytest.raises(em.EmberError) as e:
        em.Gguf(os.path.join(tmp_path, "does_not_exist.gguf"))
    assert e.value.status == em.ERR_FORMAT


def test_offsets_alignment_and_duplicates(tmp_path):
    hl = _layer()
    t = gw.moe_layer_tensors(hl, 0)
    p = _write(tmp_path, "a64.gguf", gw.moe_meta("llama", hl, 1), t, alignment=64)
    with em.Gguf(p) as g:
        assert all(x.offset % 64 == 0 for x in g.tensors())
        assert np.array_equal(g.tensor_bytes(g.find(t[1][0])), t[1][3].view(np.uint8).reshape(-1))
    _expect_format_error(tmp_path, open(_write(tmp_path, "dup.gguf", gw.moe_meta("llama", hl, 1), t + t[:1]), "rb").read(),
                         "dup2.gguf")
    # a tensor whose offset points past the end of the file
    blob = bytearray(open(p, "rb").read())
    name = t[-1][0].encode()
    at = blob.index(name) + len(name) + 4 + 8 * 3 + 4  # n_dims, ne[3], type -> offset
    blob[at:at + 8] = struct.pack("<Q", len(blob) * 2 // 64 * 64)
    _expect_format_error(tmp_path, blob, "offset.gguf")
    blob[at:at + 8] = struct.pack("<Q", 64 + 8)  # not a multiple of the alignment
    _expect_format_error(tmp_path, blob, "misaligned.gguf")


def test_nbytes():
    H = em.host()
    assert H.ember_ggml_nbytes(em.Q8_0, 64) == 68 and H.ember_ggml_nbytes(em.Q4_K, 512) == 288
    assert H.ember_ggml_nbytes(em.BF16, 3) == 6 and H.ember_ggml_nbytes(em.Q8_0, 33) == -1
    assert H.ember_ggml_nbytes(16, 256) == -1
