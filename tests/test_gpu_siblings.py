"""GPU tests of sibling linears issued concurrently on side streams (``run_concurrent``).

The concurrent calls run the same kernels on the same per-call buffers as sequential calls, so
every output must be bit-identical to the sequential one, also after later calls have allocated
and freed memory on the same streams (an output whose memory the caching allocator handed back
too early would change after the fact).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _layers(dev, shapes, seed, backend):
    from krea2_svdquant_amd.runtime.krea2_standin import random_quantized_state
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    gen = torch.Generator(device=dev).manual_seed(seed)
    return [SVDQuantLinear(random_quantized_state(n, k, rank=32, group_size=64, device=dev, generator=gen),
                           backend=backend) for n, k in shapes]


@pytest.mark.parametrize("backend", ["hip_gfx950", "hip_gfx950_w4a16"])
def test_run_concurrent_matches_sequential_bit_for_bit(dev, backend):
    from krea2_svdquant_amd.runtime.siblings import run_concurrent
    mods = _layers(dev, [(768, 512), (512, 512), (256, 512), (256, 512)], seed=21, backend=backend)
    gen_l = torch.Generator(device=dev).manual_seed(5)
    mods[2].add_lora_adapter((torch.randn(16, 512, device=dev, generator=gen_l) * 0.05).to(torch.bfloat16),
                             (torch.randn(256, 16, device=dev, generator=gen_l) * 0.05).to(torch.bfloat16),
                             scale=0.7)
    gen = torch.Generator(device=dev).manual_seed(2)
    kept = []
    for m in (300, 64, 517):                       # ragged row counts, smaller then larger
        x = torch.randn(m, 512, device=dev, generator=gen).to(torch.bfloat16)
        seq = [mod(x) for mod in mods]
        conc = run_concurrent(x, mods)
        assert [tuple(y.shape) for y in conc] == [(m, 768), (m, 512), (m, 256), (m, 256)]
        for a, b in zip(seq, conc):
            assert torch.equal(a, b)
        kept.append(([y.clone() for y in seq], conc))
        junk = [torch.randn(m, 768, device=dev) for _ in range(4)]   # churn the allocator
        del junk
    torch.cuda.synchronize()
    for seq, conc in kept:
        for a, b in zip(seq, conc):
            assert torch.equal(a, b)


def test_standin_siblings_bit_identical(dev):
    from krea2_svdquant_amd.runtime.krea2_standin import Krea2Dims, Krea2StandInTransformer
    dims = Krea2Dims(layers=2, hidden=256, heads=2, kv_heads=1, head_dim=128, mlp=512)
    model = Krea2StandInTransformer.random(dims, rank=32, group_size=64, device=dev, seed=9)
    gen = torch.Generator(device=dev).manual_seed(4)
    text = torch.randn(16, 256, device=dev, generator=gen).to(torch.bfloat16)
    latent = torch.randn(80, 256, device=dev, generator=gen).to(torch.bfloat16)
    for fused in (False, True):
        a = model.denoise_step(text, latent, dt=-0.125, fused=fused)
        b = model.denoise_step(text, latent, dt=-0.125, fused=fused, siblings=True)
        c = model.denoise_step(text, b, dt=-0.125, fused=fused, siblings=True)
        d = model.denoise_step(text, a, dt=-0.125, fused=fused)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"fused={fused}"
        assert torch.equal(c, d), f"fused={fused}"
