"""GPU tests of sibling linears issued concurrently on side streams (``run_concurrent``).

The concurrent calls run the same kernels on the same per-call buffers as sequential calls, so
every output must be bit-identical to the sequential one, also after later calls have allocated
and freed memory on the same streams (an output whose memory the caching allocator handed back
too early would change after the fact).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _layers(dev, shapes, seed, backend, group=64, rank=32):
    from krea2_svdquant_amd.runtime.krea2_standin import random_quantized_state
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    gen = torch.Generator(device=dev).manual_seed(seed)
    return [SVDQuantLinear(random_quantized_state(n, k, rank=rank, group_size=group, device=dev, generator=gen),
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


# ---- one launch for the siblings' GEMMs (svdq_w4a4_gemm_siblings) -------------------------------

def _prepared(mods, dev):
    return [m._prepare(dev, with_adapters=bool(m.lora_adapters)) for m in mods]


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("k,group", [(1024, 64), (768, 64), (1024, 128)])   # one launch (K % 512 == 0); per layer
def test_grouped_gemms_match_single_layer_forwards(dev, k, group, out_f32):
    from krea2_svdquant_amd.kernels.hip.backend import forward_prepared, forward_prepared_siblings
    # partial column tiles (160, 96), a LoRA adapter that widens one layer's rank tiles (RTp 96)
    mods = _layers(dev, [(640, k), (160, k), (384, k), (96, k)], seed=31, backend="hip_gfx950", group=group)
    gen_l = torch.Generator(device=dev).manual_seed(6)
    mods[1].add_lora_adapter((torch.randn(48, k, device=dev, generator=gen_l) * 0.05).to(torch.bfloat16),
                             (torch.randn(160, 48, device=dev, generator=gen_l) * 0.05).to(torch.bfloat16),
                             scale=0.8)
    preps = _prepared(mods, dev)
    gen = torch.Generator(device=dev).manual_seed(3)
    for m in (300, 64, 517, 256):                  # ragged row counts: partial row tiles
        x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
        single = [forward_prepared(x, p, out_f32=out_f32) for p in preps]
        for count in (4, 2, 1):
            grouped = forward_prepared_siblings(x, preps[:count], out_f32=out_f32)
            assert [tuple(y.shape) for y in grouped] == [tuple(y.shape) for y in single[:count]]
            for i, (a, b) in enumerate(zip(single, grouped)):
                assert torch.equal(a, b), f"m={m} count={count} layer {i}"


def test_grouped_gemms_at_the_block_shapes(dev):
    """to_q, to_k, to_v, to_gate at M = 4352 (2040 tiles over the XCDs) and ff.up, ff.gate, also at
    rank 64 (the reference's default MLP rank, config.py:21-23: the low-rank term in LDS chunks)."""
    from krea2_svdquant_amd.kernels.hip.backend import forward_prepared, forward_prepared_siblings
    gen = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn(4352, 6144, device=dev, generator=gen).to(torch.bfloat16)
    for shapes, seed, rank in (([(6144, 6144), (1536, 6144), (1536, 6144), (6144, 6144)], 41, 32),
                               ([(16384, 6144), (16384, 6144)], 42, 32),
                               ([(16384, 6144), (16384, 6144)], 43, 64)):
        preps = _prepared(_layers(dev, shapes, seed=seed, backend="hip_gfx950", rank=rank), dev)
        grouped = forward_prepared_siblings(x, preps)
        for i, p in enumerate(preps):
            assert torch.equal(forward_prepared(x, p), grouped[i]), f"layer {i} of {shapes}"
        del preps, grouped
        torch.cuda.empty_cache()


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("group", [64, 128])
def test_grouped_w4a16_gemms_match_single_layer_forwards(dev, group, out_f32):
    """W4A16 siblings (``svdq_w4a16_gemm_siblings``): the attention inputs at M = 2304 (one launch of
    720 tiles of 192 x 256), ragged rows and columns with a LoRA-widened layer (RTp 96 beside 32;
    one launch of 18 tiles, the grouped rounds cheaper than three launches), and two N = 6144
    layers at M = 2304 (one round of 256 x 256 tiles each beats three rounds of 192-row tiles: a
    launch per layer); every output bit-identical to the layer's own W4A16 forward."""
    from krea2_svdquant_amd.kernels.hip.backend import forward_prepared, forward_prepared_siblings
    gen = torch.Generator(device=dev).manual_seed(21 + group)
    for m, shapes, lora in ((2304, [(6144, 6144), (6144, 6144), (1536, 6144), (1536, 6144)], False),
                            (517, [(640, 1024), (160, 1024), (384, 1024)], True),
                            (2304, [(6144, 1024), (6144, 1024)], False)):
        print(f"w4a16 siblings: M={m} shapes={shapes} group={group} lora={lora} f32={out_f32}", flush=True)
        mods = _layers(dev, shapes, seed=m + group, backend="hip_gfx950_w4a16", group=group)
        if lora:
            k = shapes[1][1]
            mods[1].add_lora_adapter((torch.randn(48, k, device=dev, generator=gen) * 0.05).to(torch.bfloat16),
                                     (torch.randn(160, 48, device=dev, generator=gen) * 0.05).to(torch.bfloat16),
                                     scale=0.8)
        preps = _prepared(mods, dev)
        x = torch.randn(m, shapes[0][1], device=dev, generator=gen).to(torch.bfloat16)
        grouped = forward_prepared_siblings(x, preps, mode="w4a16", out_f32=out_f32)
        for i, p in enumerate(preps):
            assert torch.equal(forward_prepared(x, p, mode="w4a16", out_f32=out_f32), grouped[i]), f"M={m} layer {i}"
        del mods, preps, grouped
        torch.cuda.empty_cache()


def test_run_grouped_modules_and_standin(dev):
    from krea2_svdquant_amd.runtime.krea2_standin import Krea2Dims, Krea2StandInTransformer
    from krea2_svdquant_amd.runtime.siblings import run_grouped
    mods = _layers(dev, [(512, 512), (256, 512), (128, 512)], seed=51, backend="hip_gfx950")
    gen = torch.Generator(device=dev).manual_seed(12)
    x = torch.randn(2, 150, 512, device=dev, generator=gen).to(torch.bfloat16)   # leading dims kept
    for a, b in zip([m(x) for m in mods], run_grouped(x, mods)):
        assert a.shape == b.shape and torch.equal(a, b)
    w16 = _layers(dev, [(256, 512), (256, 512)], seed=52, backend="hip_gfx950_w4a16")   # W4A16 siblings
    for a, b in zip([m(x) for m in w16], run_grouped(x, w16)):
        assert torch.equal(a, b)
    dims = Krea2Dims(layers=2, hidden=512, heads=4, kv_heads=1, head_dim=128, mlp=1024)   # K % 512 == 0
    model = Krea2StandInTransformer.random(dims, rank=32, group_size=64, device=dev, seed=13)
    text = torch.randn(16, 512, device=dev, generator=gen).to(torch.bfloat16)
    latent = torch.randn(80, 512, device=dev, generator=gen).to(torch.bfloat16)
    for fused in (False, True):
        a = model.denoise_step(text, latent, dt=-0.125, fused=fused)
        b = model.denoise_step(text, latent, dt=-0.125, fused=fused, siblings="grouped")
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"fused={fused}"


@pytest.mark.parametrize("mode", ["per_layer", "shared_x"])
@pytest.mark.parametrize("group,exact", [(64, False), (128, False), (64, True)])
def test_act_quant_siblings_match_per_layer_passes(dev, group, exact, mode, monkeypatch):
    """One launch of the siblings' activation passes (and one finalize): codes, scale pairs and the
    whole mid workspace (finalized head and split partials) bit-identical to each layer's own pass;
    ranks above 32 take the per-layer path inside the C-ABI, with the same results.  shared_x: one
    workgroup runs every layer's pass over one read of x (SVDQ_ACT_SIBLINGS)."""
    monkeypatch.setenv("SVDQ_ACT_SIBLINGS", mode)
    from krea2_svdquant_amd.kernels.hip import ops
    from krea2_svdquant_amd.runtime.krea2_standin import random_quantized_state
    from krea2_svdquant_amd.kernels.hip.backend import prepare_layer
    gen = torch.Generator(device=dev).manual_seed(group + exact)
    k = 1024
    for rank, ns in ((32, (512, 128, 256, 64)), (32, (384, 256)), (64, (256, 128))):
        preps = [prepare_layer(random_quantized_state(n, k, rank=rank, group_size=group, device=dev, generator=gen))
                 for n in ns]
        rtp = preps[0].rtp
        for m in (300, 64, 4352):
            x = (torch.randn(m, k, device=dev, generator=gen) * 2).to(torch.bfloat16)
            flat = ops.act_quant_siblings(x, [p.srs for p in preps], [p.l2 for p in preps], group, rtp, exact)
            for i, p in enumerate(preps):
                qa, sx, _, _, mid = ops.act_quant(x, p.srs, p.l2, None, None, group, rtp, ops.OPERAND_E3M2, False,
                                                  False, exact, True)
                assert torch.equal(flat[3 * i], qa), f"r={rank} m={m} layer {i}: codes"
                assert torch.equal(flat[3 * i + 1], sx), f"r={rank} m={m} layer {i}: scale pairs"
                assert torch.equal(flat[3 * i + 2].view(torch.int32), mid.view(torch.int32)), \
                    f"r={rank} m={m} layer {i}: mid workspace"
