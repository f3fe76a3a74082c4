"""GPU tests of the elementwise ops fused into the GEMM store (``svdq_*_gemm_epi``).

The reference for each fused op is the same op run by torch on the GPU, on the bf16 output of
the same kernel without the op (the GEMM itself is held to the oracle by the other GPU tests):

* ``residual_gate``  ``torch.addcmul(aux, vec, y)`` (one rounding);
* ``mul_sigmoid``    ``aux * torch.sigmoid(y)``;
* ``silu_mul``       ``F.silu(aux) * y``;

each within 1 bf16 ulp and nearly all bit-equal (float evaluation order and exp may differ in the
last float bit, which can move a bf16 rounding).

Every shape class of the store is covered: the e3m2 kernel with and without its paired-stage
main loop (K % 512), the FP8 / INT8 operand kernels, both W4A16 kernels (128 x 128 tiles and the
256 x 256 tiles of large grids), N % 8 != 0 (element stores at the right edge) and M, N not
multiples of the tile.
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

OPS = ("residual_gate", "mul_sigmoid", "silu_mul")


def _layer(n, k, dev, seed):
    from krea2_svdquant_amd.kernels.hip import backend
    from krea2_svdquant_amd.runtime.krea2_standin import random_quantized_state
    gen = torch.Generator(device=dev).manual_seed(seed)
    st = random_quantized_state(n, k, device=dev, generator=gen)
    st.bias = (torch.randn(n, device=dev, generator=gen) * 0.1).to(torch.bfloat16)
    return backend.prepare_layer(st, (), dev), gen


def _torch_op(op, y, aux, vec):
    if op == "residual_gate":
        return torch.addcmul(aux, vec, y)
    if op == "mul_sigmoid":
        return aux * torch.sigmoid(y)
    return F.silu(aux) * y


def _ulp(t: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp at each element of t (the smallest normal's ulp at zero)."""
    _, e = torch.frexp(t.float())
    return torch.ldexp(torch.ones_like(t, dtype=torch.float32), torch.clamp(e - 8, min=-133))


def _check(op, fused, ref):
    assert fused.dtype == torch.bfloat16 and fused.shape == ref.shape
    diff = (fused.float() - ref.float()).abs()
    assert bool((diff <= _ulp(ref)).all()), f"{op}: max diff {float(diff.max())} beyond one bf16 ulp"
    same = float((fused == ref).float().mean())
    assert same > 0.99, f"{op}: only {same:.4f} of the elements bit-equal to torch"


@pytest.mark.parametrize("mode,operand,m,n,k", [
    ("w4a4", "e3m2", 200, 260, 512),     # paired-stage main loop, N % 8 != 0
    ("w4a4", "e3m2", 96, 130, 320),      # stage-by-stage loop with a partial stage
    ("w4a4", "e4m3", 72, 136, 256),
    ("w4a4", "i8", 40, 200, 192),
    ("w4a16", "e3m2", 64, 136, 256),     # 128 x 128 tiles
    ("w4a16", "e3m2", 512, 16384, 128),  # 192 x 256 tiles (192 of them; the last row of tiles partial)
    ("w4a16", "e3m2", 1024, 16384, 128), # 256 x 256 tiles (256 of them: 192-row tiles would need 2 rounds)
])
@pytest.mark.parametrize("op", OPS)
def test_fused_epilogue_matches_torch_op(dev, mode, operand, m, n, k, op):
    from krea2_svdquant_amd.kernels.hip import backend
    prep, gen = _layer(n, k, dev, seed=m + n + k)
    x = torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16)
    aux = torch.randn(m, n, device=dev, generator=gen).to(torch.bfloat16)
    vec = (torch.rand(n, device=dev, generator=gen) + 0.2).to(torch.bfloat16) if op == "residual_gate" else None
    y = backend.forward_prepared(x, prep, mode=mode, operand=operand)
    fused = backend.forward_prepared(x, prep, mode=mode, operand=operand, epilogue=op, aux=aux, vec=vec)
    torch.cuda.synchronize()
    _check(op, fused, _torch_op(op, y, aux, vec))


def test_fused_epilogue_takes_unaligned_views_and_leading_dims(dev):
    """aux as a view at an odd element offset (copied to an aligned buffer by the host side) and
    x / aux with leading dimensions, as a block passes them."""
    from krea2_svdquant_amd.kernels.hip import backend
    prep, gen = _layer(136, 256, dev, seed=5)
    x = torch.randn(2, 24, 256, device=dev, generator=gen).to(torch.bfloat16)
    big = torch.randn(48 * 136 + 1, device=dev, generator=gen).to(torch.bfloat16)
    aux = big[1:].view(2, 24, 136)
    assert aux.data_ptr() % 16 != 0
    vec = torch.rand(136, device=dev, generator=gen).to(torch.bfloat16)
    y = backend.forward_prepared(x, prep)
    fused = backend.forward_prepared(x, prep, epilogue="residual_gate", aux=aux, vec=vec)
    assert tuple(fused.shape) == (2, 24, 136)
    _check("residual_gate", fused, torch.addcmul(aux, vec, y))


def test_module_forward_epilogue_with_lora(dev):
    """SVDQuantLinear.forward_epilogue includes the LoRA adapters, like forward."""
    from krea2_svdquant_amd.runtime.krea2_standin import random_quantized_state
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    gen = torch.Generator(device=dev).manual_seed(9)
    mod = SVDQuantLinear(random_quantized_state(264, 512, device=dev, generator=gen), backend="hip_gfx950")
    down = (torch.randn(16, 512, device=dev, generator=gen) * 0.01).to(torch.bfloat16)
    up = (torch.randn(264, 16, device=dev, generator=gen) * 0.01).to(torch.bfloat16)
    mod.add_lora_adapter(down, up, scale=0.8)
    x = torch.randn(80, 512, device=dev, generator=gen).to(torch.bfloat16)
    g = torch.randn(80, 264, device=dev, generator=gen).to(torch.bfloat16)
    _check("silu_mul", mod.forward_epilogue(x, "silu_mul", aux=g), F.silu(g) * mod(x))


def test_fused_standin_block_matches_unfused(dev):
    """The stand-in blocks with the gates, SwiGLU and residuals fused into the linears' stores
    against the same blocks with those ops in torch (the default)."""
    from krea2_svdquant_amd.runtime.krea2_standin import Krea2Dims, Krea2StandInTransformer
    dims = Krea2Dims(layers=2, hidden=256, heads=2, kv_heads=1, head_dim=128, mlp=512)
    model = Krea2StandInTransformer.random(dims, device=dev, seed=13)
    gen = torch.Generator(device=dev).manual_seed(4)
    tokens = torch.randn(72, 256, device=dev, generator=gen).to(torch.bfloat16)
    fused = model(tokens, fused=True)
    unfused = model(tokens)
    torch.cuda.synchronize()
    err = float((fused.float() - unfused.float()).norm() / unfused.float().norm())
    same = float((fused == unfused).float().mean())
    print(f"  fused vs unfused blocks: rel_l2 {err:.3e}, bit-equal {same:.4f}")
    assert err < 5e-3 and same > 0.9


def test_fused_sigmoid_and_silu_bit_equal_to_torch_everywhere(dev):
    """The store's sigmoid / silu quotients take a reciprocal product where it rounds to the same
    bf16 as the IEEE quotient and the IEEE division elsewhere: bit-equal to torch's ops.
    silu_mul over every finite bf16 aux value (a 256 x 256 grid of all bit patterns); mul_sigmoid
    over 8M GEMM outputs of spread magnitude."""
    from krea2_svdquant_amd.kernels.hip import backend
    prep, gen = _layer(256, 128, dev, seed=21)
    bits = torch.arange(65536, dtype=torch.int32, device=dev)
    finite = (bits & 0x7F80) != 0x7F80
    aux = torch.where(finite, bits, torch.zeros_like(bits)).to(torch.int16).view(torch.bfloat16).view(256, 256)
    x = torch.randn(256, 128, device=dev, generator=gen).to(torch.bfloat16)
    y = backend.forward_prepared(x, prep)
    fused = backend.forward_prepared(x, prep, epilogue="silu_mul", aux=aux)
    ref = F.silu(aux) * y
    torch.cuda.synchronize()
    assert torch.equal(fused, ref), f"silu_mul: {int((fused != ref).sum())} elements differ from torch"

    prep, gen = _layer(16384, 128, dev, seed=22)
    x = (torch.randn(512, 128, device=dev, generator=gen) * 40).to(torch.bfloat16)
    aux = torch.randn(512, 16384, device=dev, generator=gen).to(torch.bfloat16)
    y = backend.forward_prepared(x, prep)
    fused = backend.forward_prepared(x, prep, epilogue="mul_sigmoid", aux=aux)
    ref = aux * torch.sigmoid(y)
    torch.cuda.synchronize()
    assert torch.equal(fused, ref), f"mul_sigmoid: {int((fused != ref).sum())} elements differ from torch"
