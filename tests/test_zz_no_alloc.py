"""ember_moe_ffn_noalloc (the entry point that allocates nothing and runs in the library's static
scratch) against ember_moe_ffn on the same inputs: bit-identical outputs on two calls in a row, the
second with a smaller batch, for a fused-routing decode layer, a prefill-sized MFMA layer and a layer
whose one-token call takes the slice launch; a batch
whose scratch exceeds the static buffer is refused with EMBER_ERR_SCRATCH and launches nothing."""
import numpy as np
import pytest

import ember_moe as em

pytestmark = pytest.mark.gpu


def _pair(dl, x):
    import torch

    T = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    ref, _ = dl.forward(xd)
    out = torch.full_like(xd, float("nan"))
    assert em.moe_ffn_noalloc(dl.desc, xd, T, out) == em.OK
    torch.cuda.synchronize()
    return out.cpu().numpy(), ref.cpu().numpy()


@pytest.mark.parametrize("name,spec,Ts", [
    ("q8-mixtral-like", dict(d=4096, d_ff=2048, E=8, k=2, wtype=em.Q8_0), (8, 1)),
    ("bf16-shared", dict(d=1024, d_ff=512, E=16, k=4, wtype=em.BF16, bias_std=2.0, d_ff_shared=1024), (300, 3)),
    ("f32-c1", dict(d=256, d_ff=688, E=8, k=2, wtype=em.F32), (64, 1)),
])
def test_noalloc_matches_ffn(gpu, name, spec, Ts):
    s = em.LayerSpec(seed=31, **spec)
    dl = em.DeviceLayer.upload(em.make_host_layer(s))
    for i, T in enumerate(Ts):  # the second call is smaller: stale contents of the larger one must not leak
        x = em.make_input(s, T, seed=500 + i)
        print(f"noalloc {name} call {i} T={T}", flush=True)
        got, want = _pair(dl, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, T)


def test_noalloc_slice_launch(gpu):
    """A packed Q8_0 layer whose one-token call takes the slice launch (k * d_ff / 64 = 256 slices): its
    partial rows live in the static scratch too."""
    import torch

    s = em.LayerSpec(d=1024, d_ff=8192, E=8, k=2, wtype=em.Q8_0, seed=33)
    dl = em.DeviceLayer.upload(em.make_host_layer(s))
    buf = torch.empty(em.prefill_pack_bytes(dl.desc), dtype=torch.uint8, device="cuda")
    em.prefill_pack(dl.desc, buf)
    dl.tensors["pack"] = buf
    bits = em.path(dl.desc, 1)
    if not bits & em.PATH_SLICES:
        pytest.skip(f"this device does not take the slice launch for 256 slices (path bits {bits})")
    for i, T in enumerate((8, 1)):
        x = em.make_input(s, T, seed=600 + i)
        print(f"noalloc slices call {i} T={T}", flush=True)
        got, want = _pair(dl, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), T


def test_noalloc_refuses_oversize(gpu):
    import torch

    s = em.LayerSpec(d=4096, d_ff=14336, E=8, k=2, wtype=em.BF16, seed=1)
    # descriptor only: sizing and validation need no weights, just aligned non-null pointers
    L = em.Layer()
    L.d, L.d_ff, L.E, L.k, L.renorm, L.out_scale, L.groups_n, L.groups_top = s.d, s.d_ff, s.E, s.k, 1, 1.0, 1, 1
    buf = torch.empty(1 << 12, dtype=torch.uint8, device="cuda")
    L.router = L.gate = L.up = L.down = buf.data_ptr()
    L.gate_type = L.up_type = L.down_type = em.BF16
    T = 512
    assert em.scratch_bytes(L, T) > em.NOALLOC_SCRATCH_BYTES
    x = torch.zeros((T, s.d), device="cuda")
    out = torch.full((T, s.d), 7.0, device="cuda")
    assert em.moe_ffn_noalloc(L, x, T, out) == em.ERR_SCRATCH
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)
