"""The end-to-end harness's decode attention (grouped heads, no KV repeat) against the library's fused
attention with the KV heads repeated, on the CPU in fp32."""
import pytest

torch = pytest.importorskip("torch")

from ember_moe.mixtral import Mixtral  # noqa: E402


@pytest.mark.parametrize("H,Hkv,C,D,n", [(32, 8, 48, 16, 20), (8, 8, 9, 32, 9), (6, 2, 17, 8, 1)])
def test_attend_decode_matches_repeated_kv_sdpa(H, Hkv, C, D, n):
    g = torch.Generator().manual_seed(H * 1000 + C)
    q = torch.randn(H, D, generator=g)
    kc = torch.randn(Hkv, C, D, generator=g)
    vc = torch.randn(Hkv, C, D, generator=g)
    valid = torch.arange(C) < n  # the first n cache positions hold tokens
    mbias = torch.zeros(C).masked_fill(~valid, float("-inf"))
    got = Mixtral.attend_decode(q, kc, vc, mbias)
    rep = H // Hkv
    want = torch.nn.functional.scaled_dot_product_attention(
        q[None, :, None, :], kc.repeat_interleave(rep, 0)[None], vc.repeat_interleave(rep, 0)[None],
        attn_mask=valid[None, None, None, :])[0, :, 0, :]
    assert got.shape == (H, D)
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-5), (got - want).abs().max()



def test_rope_matrix_equals_rotate_half():
    D, hd = 16, 8
    g = torch.Generator().manual_seed(5)
    x = torch.randn(6, D, generator=g)
    ang = torch.randn(hd, generator=g)
    cos, sin = torch.cat([ang.cos(), ang.cos()]), torch.cat([ang.sin(), ang.sin()])
    perm = Mixtral.rope_perm(D)
    assert torch.equal(x @ perm, torch.cat([-x[:, hd:], x[:, :hd]], -1))
    want = Mixtral._rot(x, cos, sin)
    got = x @ Mixtral.rot_matrix(cos, sin, perm)
    assert torch.allclose(got, want, rtol=1e-6, atol=1e-6)
