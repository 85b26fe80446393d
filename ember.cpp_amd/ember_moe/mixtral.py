"""End-to-end Mixtral-architecture harness around the MoE FFN C ABI.

A random-init Mixtral-8x7B-shaped decoder (token embedding, RMSNorm, GQA attention with RoPE and a KV
cache, the MoE FFN, final norm and LM head) runs a seeded prompt prefill and greedy decode steps at
batch 1. Only the MoE FFN is this project's path: every layer's FFN is one ember_moe_ffn call on expert
stacks held in their ggml encoding (Q4_K by default), as model.cpp's MoE branch would call it
(model.cpp:2821-2827). Attention, norms, embeddings and the head are plain PyTorch (bf16 matmuls,
fp32 residual stream): they stand in for the reference's engine, which is outside the built path.

Decode steps are captured once in a HIP graph (static shapes: the KV cache has a fixed capacity, the
position lives on the device and drives the RoPE gather, the cache write and the attention mask) and
replayed per token, so a step costs its kernels, not Python.

Weights: experts N(0, 0.02) quantized with the repo's quantizer; `expert_sets` distinct sets are
generated (host quantization of 45 B parameters would take minutes) and every layer holds its own
device copy of one of them, so no two layers share memory. Attention and head weights are bf16
N(0, 0.02) (the reference's config quantizes them to Q4_K as well; here they are torch GEMM operands),
norms are ones, routers F32 N(0, 1/sqrt(d)).
"""
from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np

from . import (EmberError, Layer, Q4_K, TYPE_NAMES, _ptr, moe_ffn, prefill_pack, prefill_pack_bytes, quantize,
               scratch_bytes)


@dataclass
class MixtralSpec:
    n_layers: int = 32
    d: int = 4096
    n_heads: int = 32
    n_kv: int = 8
    head_dim: int = 128
    E: int = 8
    k: int = 2
    d_ff: int = 14336
    vocab: int = 32000
    rope_theta: float = 1e6
    eps: float = 1e-5
    expert_type: int = Q4_K
    expert_sets: int = 4
    seed: int = 0
    prefill_pack: bool = True  # each layer's experts also repacked for the prefill tile GEMMs (ember_moe_prefill_pack)


class Mixtral:
    def __init__(self, spec: MixtralSpec, max_ctx: int, device="cuda", log=print):
        import torch

        self.s, self.max_ctx, self.dev = spec, max_ctx, device
        s = spec
        g = torch.Generator(device=device)
        g.manual_seed(s.seed)

        def randn(*shape, std=0.02, dtype=torch.bfloat16):
            return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(dtype)

        t0 = time.time()
        self.emb = randn(s.vocab, s.d)
        self.head = randn(s.vocab, s.d)
        qd, kvd = s.n_heads * s.head_dim, s.n_kv * s.head_dim
        self.wqkv = [randn(qd + 2 * kvd, s.d) for _ in range(s.n_layers)]
        self.wo = [randn(s.d, qd) for _ in range(s.n_layers)]
        self.routers = [randn(s.E, s.d, std=1.0 / np.sqrt(s.d), dtype=torch.float32) for _ in range(s.n_layers)]
        # expert stacks: normals drawn on the device, quantized on the host, one device copy per layer
        sets = []
        for i in range(min(s.expert_sets, s.n_layers)):
            mats = []
            for shape in ((s.E, s.d_ff, s.d), (s.E, s.d_ff, s.d), (s.E, s.d, s.d_ff)):
                w = randn(*shape, dtype=torch.float32).cpu().numpy().reshape(-1)
                mats.append(torch.from_numpy(quantize(s.expert_type, w)).to(device))
            sets.append(mats)
        self.experts, self.layers, self.packs = [], [], []
        for l in range(s.n_layers):
            gate, up, down = (m.clone() for m in sets[l % len(sets)])
            L = Layer()
            L.d, L.d_ff, L.E, L.k = s.d, s.d_ff, s.E, s.k
            L.renorm, L.scoring, L.groups_n, L.groups_top, L.out_scale = 1, 0, 1, 1, 1.0
            L.router = _ptr(self.routers[l])
            L.gate, L.gate_type = _ptr(gate), s.expert_type
            L.up, L.up_type = _ptr(up), s.expert_type
            L.down, L.down_type = _ptr(down), s.expert_type
            if s.prefill_pack and prefill_pack_bytes(L) > 0:
                buf = torch.empty(prefill_pack_bytes(L), dtype=torch.uint8, device=device)
                prefill_pack(L, buf)
                self.packs.append(buf)
            self.experts.append((gate, up, down))
            self.layers.append(L)
        del sets
        torch.cuda.synchronize()
        self.expert_bytes = sum(sum(t.numel() for t in e) for e in self.experts)
        self.pack_bytes = sum(t.numel() for t in self.packs)
        log(f"[e2e] weights ready in {time.time() - t0:.1f}s: {s.n_layers} layers, experts "
            f"{TYPE_NAMES[s.expert_type]} {self.expert_bytes / 1e9:.1f} GB (+ prefill packs {self.pack_bytes / 1e9:.1f} GB)")
        # RoPE tables (rotate-half pairing) and the KV cache
        inv = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2, device=device, dtype=torch.float64) / s.head_dim))
        ang = torch.arange(max_ctx, device=device, dtype=torch.float64)[:, None] * inv[None, :]
        self.cos = torch.cat([ang.cos(), ang.cos()], -1).float()
        self.sin = torch.cat([ang.sin(), ang.sin()], -1).float()
        # decode: RoPE as one matmul by a per-position [D, D] matrix (rot_matrix), built once per step
        self.rot_perm = self.rope_perm(s.head_dim, device)
        self.kcache = torch.zeros(s.n_layers, s.n_kv, max_ctx, s.head_dim, device=device, dtype=torch.bfloat16)
        self.vcache = torch.zeros_like(self.kcache)
        self.scratch = None
        # optional hook probe(layer, h, f, scratch, layer_descriptor) after every eager MoE FFN call (the
        # per-layer parity check of the end-to-end test reads the call's inputs, output and routing)
        self.probe = None

    # ---- pieces
    def _rms(self, x):
        import torch.nn.functional as F

        # x / sqrt(mean(x^2) + eps), in one library call (the stand-in model has no norm weights)
        return F.rms_norm(x, (x.shape[-1],), eps=self.s.eps)

    @staticmethod
    def _rot(x, cos, sin):
        import torch

        h = x.shape[-1] // 2
        return x * cos + torch.cat([-x[..., h:], x[..., :h]], -1) * sin

    def _attend(self, q, k, v, mask=None, causal=False):
        import torch.nn.functional as F

        try:
            return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal, enable_gqa=True)
        except TypeError:
            rep = self.s.n_heads // self.s.n_kv
            return F.scaled_dot_product_attention(q, k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1),
                                                  attn_mask=mask, is_causal=causal)

    @staticmethod
    def rope_perm(D, device="cpu"):
        """The signed rotate-half permutation: x @ P = rotate_half(x) = [-x[D/2:], x[:D/2]]."""
        import torch

        hd = D // 2
        P = torch.zeros(D, D, device=device)
        P[torch.arange(hd) + hd, torch.arange(hd)] = -1.0  # out[j] = -x[j + D/2], j < D/2
        P[torch.arange(hd), torch.arange(hd) + hd] = 1.0   # out[j] = x[j - D/2], j >= D/2
        return P

    @staticmethod
    def rot_matrix(cos, sin, perm):
        """R with x @ R = x cos + rotate_half(x) sin for one position (cos, sin [D]; perm the signed
        rotate-half permutation, perm[i][j] = -1 for i = j + D/2, 1 for j = i + D/2)."""
        import torch

        return torch.diag(cos) + perm * sin[None, :]

    @staticmethod
    def attend_decode(q, kc, vc, mbias):
        """One token's grouped-query attention over a KV cache without repeating the KV heads: q [H, D]
        (head h reads KV head h // (H / Hkv)), kc / vc [Hkv, C, D], mbias [C] an additive mask (0 for the
        cache positions that hold tokens, -inf elsewhere); returns [H, D]. Everything runs in the cache's
        dtype except the softmax, which accumulates in fp32. (The fused scaled_dot_product_attention call
        with a boolean mask and grouped heads showed three ~20 us device-to-device copies per layer and
        step in a kernel trace of the decode graph; this form is five kernels.)"""
        import torch

        H, D = q.shape
        Hkv = kc.shape[0]
        qg = q.reshape(Hkv, H // Hkv, D).to(kc.dtype)
        sc = torch.add(mbias, torch.matmul(qg, kc.transpose(1, 2)), alpha=1.0 / D ** 0.5)
        return torch.matmul(torch.softmax(sc, -1), vc).reshape(H, D)

    def _moe(self, l, h, T):
        import torch

        f = torch.empty_like(h)
        st = moe_ffn(self.layers[l], h, T, f, self.scratch)
        if st:
            raise EmberError(st, "ember_moe_ffn")
        if self.probe is not None:
            self.probe(l, h, f, self.scratch, self.layers[l])
        return f

    def _ensure_scratch(self, T):
        import torch

        # (decode steps run T = 1 calls in the same buffer, whose one-token path has sections of its own)
        need = max(scratch_bytes(L, n) for L in self.layers[:1] for n in (T, 1))
        if need == 0:
            raise EmberError(-1, "ember_moe_scratch_bytes")
        if self.scratch is None or self.scratch.numel() < need:
            self.scratch = torch.empty(need, dtype=torch.uint8, device=self.dev)

    # ---- prefill: T tokens at positions [0, T)
    def prefill(self, tokens):
        import torch

        s = self.s
        T = tokens.numel()
        self._ensure_scratch(T)
        x = self.emb[tokens].float()
        cos, sin = self.cos[:T], self.sin[:T]
        qd, kvd = s.n_heads * s.head_dim, s.n_kv * s.head_dim
        for l in range(s.n_layers):
            h = self._rms(x).to(torch.bfloat16)
            qkv = (h @ self.wqkv[l].t()).float()
            qk = self._rot(qkv[:, :qd + kvd].view(T, s.n_heads + s.n_kv, s.head_dim), cos[:, None], sin[:, None])
            q, k = qk[:, :s.n_heads], qk[:, s.n_heads:]
            v = qkv[:, qd + kvd:].view(T, s.n_kv, s.head_dim)
            self.kcache[l, :, :T] = k.transpose(0, 1).to(torch.bfloat16)
            self.vcache[l, :, :T] = v.transpose(0, 1).to(torch.bfloat16)
            a = self._attend(q.transpose(0, 1)[None].to(torch.bfloat16), self.kcache[l, :, :T][None],
                             self.vcache[l, :, :T][None], causal=True)
            x = x + (a[0].transpose(0, 1).reshape(T, qd) @ self.wo[l].t()).float()
            x = x + self._moe(l, self._rms(x).contiguous(), T)
        logits = self._rms(x[-1:]).to(torch.bfloat16) @ self.head.t()
        return logits.float().argmax(-1)

    # ---- one decode step at device position pos (int64 [1]), token tok (int64 [1]); in place
    def _decode_step(self, tok, pos, out_tokens, first_pos, skip_moe=False):
        import torch

        s = self.s
        qd, kvd = s.n_heads * s.head_dim, s.n_kv * s.head_dim
        x = self.emb[tok].float()
        rot = self.rot_matrix(self.cos[pos][0], self.sin[pos][0], self.rot_perm).to(torch.bfloat16)
        mbias = torch.zeros(self.max_ctx, device=self.dev, dtype=torch.bfloat16)
        mbias.masked_fill_(torch.arange(self.max_ctx, device=self.dev) > pos, float("-inf"))
        for l in range(s.n_layers):
            h = self._rms(x).to(torch.bfloat16)
            qkv = h @ self.wqkv[l].t()  # bf16: q, k, v and their rotation stay in the cache's dtype
            qk = (qkv[:, :qd + kvd].view(s.n_heads + s.n_kv, s.head_dim) @ rot)[None]
            q, k = qk[:, :s.n_heads], qk[:, s.n_heads:]
            v = qkv[:, qd + kvd:].view(1, s.n_kv, s.head_dim)
            self.kcache[l].index_copy_(1, pos, k.transpose(0, 1))
            self.vcache[l].index_copy_(1, pos, v.transpose(0, 1))
            a = self.attend_decode(q[0], self.kcache[l], self.vcache[l], mbias)
            x = x + (a.reshape(1, qd) @ self.wo[l].t()).float()
            if not skip_moe:
                x = x + self._moe(l, self._rms(x).contiguous(), 1)
        nxt = (self._rms(x).to(torch.bfloat16) @ self.head.t()).float().argmax(-1)
        out_tokens.index_copy_(0, pos - first_pos, nxt)
        tok.copy_(nxt)
        pos.add_(1)

    def generate(self, prompt, n_new, use_graph=True, skip_moe=False):
        """Prefill `prompt` (int64 device tensor), then n_new greedy decode steps. Returns (the token the
        prefill predicts, the n_new tokens the decode steps predict, prefill seconds, decode seconds).
        skip_moe: decode steps without the MoE FFN calls (to measure the FFN's share of a step)."""
        import torch

        T = prompt.numel()
        assert T + n_new <= self.max_ctx
        torch.cuda.synchronize()
        t0 = time.time()
        first = self.prefill(prompt)
        torch.cuda.synchronize()
        t_prefill = time.time() - t0
        self._ensure_scratch(T)
        tok = first.clone().view(1)
        pos = torch.full((1,), T, dtype=torch.int64, device=self.dev)
        out = torch.zeros(n_new, dtype=torch.int64, device=self.dev)
        if use_graph:
            # capture one step (warm it first on a side stream: allocations happen outside the graph)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            saved = (tok.clone(), pos.clone(), self.kcache.clone(), self.vcache.clone())
            with torch.cuda.stream(side):
                self._decode_step(tok, pos, out, T, skip_moe)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._decode_step(tok, pos, out, T, skip_moe)
            tok.copy_(saved[0]); pos.copy_(saved[1]); self.kcache.copy_(saved[2]); self.vcache.copy_(saved[3])
            del saved
            torch.cuda.synchronize()
            t1 = time.time()
            for _ in range(n_new):
                graph.replay()
            torch.cuda.synchronize()
            t_decode = time.time() - t1
        else:
            torch.cuda.synchronize()
            t1 = time.time()
            for _ in range(n_new):
                self._decode_step(tok, pos, out, T, skip_moe)
            torch.cuda.synchronize()
            t_decode = time.time() - t1
        return first.view(1), out, t_prefill, t_decode
