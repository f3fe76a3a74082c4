"""GPU tests of the W4A4 GEMM's two tilings: 256 x 128 blocks and 256 x 256 blocks.

Both run the same per-output arithmetic (group sums on the FP6 MFMA, scale products on the bf16
MFMA, the rescale FMAs in group order, the same epilogue), so a shape run on either tiling must give
bit-identical outputs.  ``SVDQ_W4A4_TILES`` forces one tiling; the wide tiles need M, N and K
multiples of 256.  The automatic choice at the benchmark shapes (ff.up takes the wide tiles) is
covered against the oracle by ``test_gpu_e3m2_shapes.py``.
"""
import os
from contextlib import contextmanager

import pytest
import torch

pytestmark = pytest.mark.gpu


@contextmanager
def _tiles(policy):
    old = os.environ.get("SVDQ_W4A4_TILES")
    os.environ["SVDQ_W4A4_TILES"] = policy
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("SVDQ_W4A4_TILES", None)
        else:
            os.environ["SVDQ_W4A4_TILES"] = old


def _layers(dev, shapes, seed, bias=False, ranks=None):
    from krea2_svdquant_amd.runtime.krea2_standin import random_quantized_state
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    gen = torch.Generator(device=dev).manual_seed(seed)
    mods = []
    for i, (n, k) in enumerate(shapes):
        rank = ranks[i] if ranks else 32
        st = random_quantized_state(n, k, rank=rank, group_size=64, device=dev, generator=gen)
        if bias:
            st.bias = (torch.randn(n, device=dev, generator=gen) * 0.1).to(torch.bfloat16)
        mods.append(SVDQuantLinear(st, backend="hip_gfx950"))
    return mods


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("m,n,k,lora", [(256, 256, 256, False), (512, 768, 512, False), (1024, 512, 1536, True),
                                        (768, 1024, 2048, False)])
def test_wide_tiles_bit_identical_to_narrow(dev, m, n, k, lora, out_f32):
    from krea2_svdquant_amd.kernels.hip.backend import forward_prepared
    mod = _layers(dev, [(n, k)], seed=m + n + k, bias=True)[0]
    if lora:   # LoRA ranks 64 + 32 on the rank-32 branch: RTp 128, the low-rank term in LDS chunks
        gen = torch.Generator(device=dev).manual_seed(7)
        for r in (64, 32):
            mod.add_lora_adapter((torch.randn(r, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16),
                                 (torch.randn(n, r, device=dev, generator=gen) * 0.02).to(torch.bfloat16), scale=0.8)
    prep = mod._prepare(dev, with_adapters=bool(mod.lora_adapters))
    gen = torch.Generator(device=dev).manual_seed(11)
    x = (torch.randn(m, k, device=dev, generator=gen) * 2).to(torch.bfloat16)
    x[:, ::97] *= 20   # outlier channels
    with _tiles("256x128"):
        a = forward_prepared(x, prep, out_f32=out_f32)
    with _tiles("256x256"):
        b = forward_prepared(x, prep, out_f32=out_f32)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("ranks", [None, (64, 32, 64)])
def test_wide_tiles_siblings_bit_identical(dev, out_f32, ranks):
    """Sibling launches on both tilings against a launch per layer; ranks (64, 32, 64) take the
    low-rank term in LDS chunks for every layer of the launch (the rank-32 one in a single chunk)."""
    from krea2_svdquant_amd.kernels.hip.backend import forward_prepared, forward_prepared_siblings
    mods = _layers(dev, [(768, 1024), (256, 1024), (512, 1024)], seed=23, ranks=ranks)
    preps = [m._prepare(dev, with_adapters=False) for m in mods]
    gen = torch.Generator(device=dev).manual_seed(13)
    x = torch.randn(512, 1024, device=dev, generator=gen).to(torch.bfloat16)
    with _tiles("256x128"):
        narrow = forward_prepared_siblings(x, preps, out_f32=out_f32)
        single = [forward_prepared(x, p, out_f32=out_f32) for p in preps]
    with _tiles("256x256"):
        wide = forward_prepared_siblings(x, preps, out_f32=out_f32)
    torch.cuda.synchronize()
    for i, (a, b, c) in enumerate(zip(narrow, wide, single)):
        assert torch.equal(a, b), f"layer {i}"
        assert torch.equal(a, c), f"layer {i}"
