"""GPU tests of the module boundary (SVDQuantLinear) and benchmark-sized layers."""
import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sim, synth
from tests.gpu_util import (bf16_bits_of, bf16_tensor, from_device_state, operand_bytes, rel_l2,
                            to_device_state)

pytestmark = pytest.mark.gpu


def test_module_forward_with_lora_matches_oracle(dev):
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    x = synth.make_activation(96, 1024, seed=31)
    st = synth.make_layer(384, 1024, x, rank=32, group_size=64, seed=32, bias=True)
    mod = SVDQuantLinear(to_device_state(st, dev), backend="auto")
    y0 = mod(bf16_tensor(x, dev).reshape(2, 48, 1024))
    assert tuple(y0.shape) == (2, 48, 384) and y0.dtype == torch.bfloat16
    ref0 = sim.w4a4_eval(x, st)["y"]
    assert rel_l2(y0.float().cpu().numpy().reshape(96, 384), nm.bf16(ref0.astype(np.float32))) < 1e-3
    ad = synth.make_adapter(384, 1024, rank=64, seed=33, scale=0.8)
    mod.add_lora_adapter(bf16_tensor(ad.down, dev), bf16_tensor(ad.up, dev), scale=0.8)
    st.adapters.append(ad)
    y1 = mod(bf16_tensor(x, dev))
    ref1 = sim.w4a4_eval(x, st)["y"]
    assert rel_l2(y1.float().cpu().numpy(), nm.bf16(ref1.astype(np.float32))) < 1e-3
    # _forward_base excludes adapters, as in the reference
    yb = mod._forward_base(bf16_tensor(x, dev))
    assert torch.equal(yb, y0.reshape(96, 384))


def test_backend_function_matches_module_and_reuses_operands(dev):
    """The stateless backend function (reference seam ``fn(x, state)``) gives the module's output
    bit for bit and prepares the state once."""
    from krea2_svdquant_amd.kernels.hip import backend
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    x = synth.make_activation(80, 512, seed=35)
    st = synth.make_layer(192, 512, x, rank=32, group_size=64, seed=36, bias=True)
    ds = to_device_state(st, dev)
    xd = bf16_tensor(x, dev)
    y_mod = SVDQuantLinear(ds, backend="hip_gfx950")(xd)
    y1 = backend.svdquant_linear_hip_gfx950(xd, ds)
    prep = backend._SEAM_CACHE[id(ds)][1]
    y2 = backend.svdquant_linear_hip_gfx950(xd, ds)
    assert backend._SEAM_CACHE[id(ds)][1] is prep and prep.operands
    assert torch.equal(y1, y_mod) and torch.equal(y2, y_mod)


def test_w4a16_module_matches_sim_math(dev):
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    x = synth.make_activation(64, 512, seed=41)
    st = synth.make_layer(256, 512, x, rank=32, group_size=64, seed=42, bias=True)
    mod = SVDQuantLinear(to_device_state(st, dev), backend="hip_gfx950_w4a16")
    y = mod(bf16_tensor(x, dev)).float().cpu().numpy()
    ref = sim.w4a16_eval(x, st)["y"]
    assert rel_l2(y, nm.bf16(ref.astype(np.float32))) < 1e-3
    y_sim = sim.sim_forward_torch(torch.from_numpy(x).to(torch.bfloat16), st).float().numpy()
    assert rel_l2(y, y_sim) < 1e-2   # the reference sim rounds mid and every sum to bf16


def test_config0_layer(dev):
    """benchmark config 0 shape: M=256, K=N=6144, rank 32, group 64, outlier channels."""
    from krea2_svdquant_amd.kernels.hip import backend
    x = synth.make_activation(256, 6144, seed=0)
    st = synth.make_layer(6144, 6144, x, rank=32, group_size=64, seed=1)
    prep = backend.prepare_layer(to_device_state(st, dev), (), dev)
    xd = bf16_tensor(x, dev)
    r = sim.w4a4_eval(x, st)
    for operand in ("e4m3", "i8"):
        y32 = backend.forward_prepared(xd, prep, mode="w4a4", out_f32=True, operand=operand).cpu().numpy()
        e = rel_l2(y32, r["y"])
        print(f"  config0 w4a4/{operand} rel_l2={e:.3e}")
        assert e < 1e-4
    y16 = backend.forward_prepared(xd, prep, mode="w4a16", out_f32=True).cpu().numpy()
    e16 = rel_l2(y16, sim.w4a16_eval(x, st)["y"])
    print(f"  config0 w4a16 rel_l2={e16:.3e}")
    assert e16 < 1e-4


def test_full_size_ffup_codes_exact_and_rows_sampled(dev):
    """Config 1 ff.up at full size (M=4096, K=6144, N=16384): every activation code and scale
    bit-exact, a row sample of the layer output against float64, and the exact power-of-two
    homogeneity y(2x) - b = 2 (y(x) - b) over the whole output."""
    from krea2_svdquant_amd.kernels.hip import backend, ops
    from krea2_svdquant_amd.quant.convert import convert_linear
    torch.manual_seed(0)
    m, k, n = 4096, 6144, 16384
    x = synth.make_activation(m, k, seed=0)
    xd = bf16_tensor(x, dev)
    w = torch.randn(n, k, device=dev) * 0.02
    ds = convert_linear(w, torch.randn(n, device=dev) * 0.1, xd.float().abs().amax(0), rank=32,
                        group_size=64, smooth_clamp=(None, None), seed=3)
    del w
    prep = backend.prepare_layer(ds, (), dev)
    qa, sx, qx, _, mid = ops.act_quant(xd, prep.srs, prep.l2, None, None, 64, prep.rtp, ops.OPERAND_E4M3,
                                       True, False, False)
    st = from_device_state(ds)
    xh, packed, sxo, codes = sim.quantize_activations(x, st)
    assert np.array_equal(qx.cpu().numpy(), packed)
    assert np.array_equal(qa.cpu().numpy(), operand_bytes(codes, "e4m3"))
    assert np.array_equal(bf16_bits_of(sx), nm.bf16_bits(sxo))
    y = backend.forward_prepared(xd, prep, mode="w4a4", out_f32=True)
    rows = np.random.default_rng(1).choice(m, 48, replace=False)
    r = sim.w4a4_eval(x[rows], st)
    e = rel_l2(y[torch.from_numpy(rows).to(dev)].cpu().numpy(), r["y"])
    print(f"  ff.up sampled rel_l2={e:.3e}")
    assert e < 1e-4
    y2 = backend.forward_prepared(xd * 2, prep, mode="w4a4", out_f32=True)
    b = ds.bias.float()
    hom = ((y2 - b) - 2 * (y - b)).norm() / (y - b).norm()
    assert hom.item() < 1e-6


def test_checkpoint_and_lora_loaders_end_to_end(dev, tmp_path):
    """Dense model -> converter (SVD and quantization on the GPU) -> safetensors checkpoint ->
    reader into a fresh model -> LoRA file -> fused forward of every loaded layer, each against
    the oracle evaluation of the state the reader built (with the loaded adapter)."""
    from torch import nn
    from safetensors.torch import save_file
    from krea2_svdquant_amd.quant.checkpoint import convert_transformer
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    from krea2_svdquant_amd.runtime.load import load_svdquant_transformer
    from krea2_svdquant_amd.runtime.lora import load_svdquant_lora_adapters

    def dense(seed):
        torch.manual_seed(seed)
        root = nn.Module()
        blk = nn.Module()
        blk.attn = nn.Module()
        blk.attn.to_q = nn.Linear(512, 384)
        blk.attn.to_k = nn.Linear(512, 128, bias=False)
        blk.ff = nn.Module()
        blk.ff.up = nn.Linear(512, 640, bias=False)
        for lin in (blk.attn.to_q, blk.attn.to_k, blk.ff.up):
            nn.init.normal_(lin.weight, std=0.02)
        root.transformer_blocks = nn.ModuleList([blk])
        return root

    x = synth.make_activation(80, 512, seed=51)
    absmax = {"transformer_blocks.0.attn.to_q": torch.from_numpy(np.abs(x).max(0)),
              "transformer_blocks.0.ff.up": torch.from_numpy(np.abs(x).max(0))}
    meta = convert_transformer(dense(50), tmp_path / "ckpt", absmax=absmax, group_size=64, attn_rank=32,
                               mlp_rank=64, svd_device=dev, seed=7, log=None)
    assert set(meta["layers"]) == {"transformer_blocks.0.attn.to_q", "transformer_blocks.0.attn.to_k",
                                   "transformer_blocks.0.ff.up"}
    model = dense(99)
    rep = load_svdquant_transformer(model, tmp_path / "ckpt", backend="auto")["_load_report"]
    assert len(rep["replaced"]) == 3 and not rep["missing"]
    model.to(dev)
    ad = synth.make_adapter(384, 512, rank=16, seed=52)
    save_file({"transformer.transformer_blocks.0.attn.to_q.lora_A.weight": torch.from_numpy(ad.down).to(torch.bfloat16),
               "transformer.transformer_blocks.0.attn.to_q.lora_B.weight": torch.from_numpy(ad.up).to(torch.bfloat16),
               "transformer.transformer_blocks.0.attn.to_q.alpha": torch.tensor(8.0)}, tmp_path / "lora.safetensors")
    lrep = load_svdquant_lora_adapters(model, tmp_path / "lora.safetensors", scale=0.8)
    assert lrep["loaded"] == ["transformer_blocks.0.attn.to_q"]
    xd = bf16_tensor(x, dev)
    blk = model.transformer_blocks[0]
    for mod, adapters in ((blk.attn.to_q, [sim.Adapter(ad.down, ad.up, scale=0.8, network_alpha=8.0)]),
                          (blk.attn.to_k, []), (blk.ff.up, [])):
        assert isinstance(mod, SVDQuantLinear)
        y = mod(xd).float().cpu().numpy()
        st = from_device_state(mod.state)
        st.adapters.extend(adapters)
        e = rel_l2(y, nm.bf16(sim.w4a4_eval(x, st)["y"].astype(np.float32)))
        print(f"  loaded {tuple(st.shape)} adapters={len(adapters)} rel_l2={e:.3e}")
        assert e < 1e-3
