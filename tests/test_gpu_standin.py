"""GPU tests of the stand-in Krea-2 denoiser (whole blocks on the gfx950 linears).

Block outputs are checked in two independent parts, so that neither hides behind the other:

* every quantized linear the GPU forward calls is recorded with its own bf16 input and held to
  the float64 W4A4 oracle on that input (rel-L2 <= 1e-3 against bf16(oracle)): the kernels see
  the activations of a real block (post-norm, post-attention, SwiGLU products), not only
  synthetic Gaussians;
* the glue around the linears (norms, rotary embedding, GQA attention, gates, residuals) is
  replayed on the CPU in float32 with the recorded linear outputs fed back in, and the block
  outputs are compared (bf16 intermediates on the GPU: rel-L2 <= 2e-2).

A free-running CPU reference of the whole block would differ by 4-bit code flips (a bf16
difference in a linear's input moves some activation codes by one step), which no useful
tolerance separates from a real error.
"""
import numpy as np
import pytest
import torch

from oracle import numerics as nm
from oracle import sim
from tests.gpu_util import from_device_state, rel_l2

pytestmark = pytest.mark.gpu


def _small_model(dev, layers=2, seed=7):
    from krea2_svdquant_amd.runtime.krea2_standin import Krea2Dims, Krea2StandInTransformer
    dims = Krea2Dims(layers=layers, hidden=256, heads=2, kv_heads=1, head_dim=128, mlp=512)
    return Krea2StandInTransformer.random(dims, rank=32, group_size=64, device=dev, seed=seed)


def test_standin_blocks_linears_and_glue(dev):
    from krea2_svdquant_amd.runtime import krea2_standin as ks
    model = _small_model(dev)
    gen = torch.Generator(device=dev).manual_seed(3)
    text = torch.randn(16, 256, device=dev, generator=gen).to(torch.bfloat16)
    latent = torch.randn(64, 256, device=dev, generator=gen).to(torch.bfloat16)
    tokens = torch.cat([text, latent], 0)

    calls = []

    def record(name, mod, x):
        y = mod(x)
        calls.append((mod, x.detach().clone(), y.detach().clone()))
        return y

    out = model(tokens, linear=record)
    torch.cuda.synchronize()
    assert out.shape == tokens.shape and out.dtype == torch.bfloat16
    assert torch.isfinite(out.float()).all()
    assert len(calls) == 8 * len(model.transformer_blocks)

    # (1) each linear against the oracle on its recorded input
    states = {}
    for mod, x, y in calls:
        st = states.setdefault(id(mod), from_device_state(mod.state))
        ref = sim.w4a4_eval(x.float().cpu().numpy(), st)["y"]
        err = rel_l2(y.float().cpu().numpy(), nm.bf16(ref.astype(np.float32)))
        assert err < 1e-3, f"linear {tuple(st.shape)}: rel_l2 {err}"

    # (2) the glue, replayed on the CPU in float32 with the recorded linear outputs
    outputs = iter([y.float().cpu() for _, _, y in calls])

    def replay(name, mod, x):
        return next(outputs)

    x = tokens.float().cpu()
    cos, sin = ks.rope_tables(x.shape[0], 128, "cpu", torch.float32)
    for blk in model.transformer_blocks:
        x = blk(x, cos, sin, replay, modulation=blk.modulation.float().cpu())
    err = rel_l2(out.float().cpu().numpy(), x.numpy())
    assert err < 2e-2, f"block glue rel_l2 {err}"


def test_denoise_step_matches_forward_and_is_deterministic(dev):
    model = _small_model(dev, layers=1, seed=11)
    gen = torch.Generator(device=dev).manual_seed(5)
    text = torch.randn(8, 256, device=dev, generator=gen).to(torch.bfloat16)
    latent = torch.randn(40, 256, device=dev, generator=gen).to(torch.bfloat16)
    a = model.denoise_step(text, latent, dt=-0.125)
    b = model.denoise_step(text, latent, dt=-0.125)
    assert torch.equal(a, b)
    v = model(torch.cat([text, latent], 0))[8:]
    assert torch.equal(a, latent + (-0.125) * v)


def test_standin_module_names_follow_reference_targets(dev):
    from krea2_svdquant_amd.config import SVDQuantConfig
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    model = _small_model(dev, layers=1)
    names = [n for n, m in model.named_modules() if isinstance(m, SVDQuantLinear)]
    assert names == [f"transformer_blocks.0.{t}" for t in SVDQuantConfig().target_modules]
