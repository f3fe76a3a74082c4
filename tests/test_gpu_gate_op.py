"""GPU tests of ``svdq::gate_op`` (``svdq_gate_op``): the block's sigmoid output gate and SwiGLU
product as one pass each, bit-equal to the torch ops on bf16 tensors.

The op code is the GEMM store's (its reciprocal-product quotient is taken only where it rounds to
the IEEE quotient's bf16), so the reference is torch itself: ``aux * torch.sigmoid(y)`` and
``F.silu(aux) * y``.  Inputs cover every finite bf16 bit pattern on the sigmoid / silu argument,
spread magnitudes on the other operand, sizes that are not multiples of the 8-element chunk
(the tail path), unaligned views (copied to aligned buffers) and in-place use through the C-ABI.
"""
import ctypes

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _every_finite_bf16(dev):
    bits = torch.arange(65536, dtype=torch.int32, device=dev)
    finite = (bits & 0x7F80) != 0x7F80
    return torch.where(finite, bits, torch.zeros_like(bits)).to(torch.int16).view(torch.bfloat16)


def test_gate_ops_bit_equal_to_torch_over_every_finite_argument(dev):
    from krea2_svdquant_amd.kernels.hip import ops
    gen = torch.Generator(device=dev).manual_seed(31)
    arg = _every_finite_bf16(dev).view(256, 256)
    other = (torch.randn(256, 256, device=dev, generator=gen) * 30).to(torch.bfloat16)
    got = ops.gate_op(other, arg, ops.EPILOGUES["silu_mul"])        # silu(arg) * other
    ref = F.silu(arg) * other
    torch.cuda.synchronize()
    assert torch.equal(got, ref), f"silu_mul: {int((got != ref).sum())} elements differ"
    got = ops.gate_op(arg, other, ops.EPILOGUES["mul_sigmoid"])     # other * sigmoid(arg)
    ref = other * torch.sigmoid(arg)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), f"mul_sigmoid: {int((got != ref).sum())} elements differ"


@pytest.mark.parametrize("shape", [(4352, 16384), (7,), (3, 13), (1000, 6147)])
def test_gate_ops_sizes_and_tails(dev, shape):
    from krea2_svdquant_amd.kernels.hip import ops
    gen = torch.Generator(device=dev).manual_seed(sum(shape))
    y = (torch.randn(*shape, device=dev, generator=gen) * 4).to(torch.bfloat16)
    aux = (torch.randn(*shape, device=dev, generator=gen) * 4).to(torch.bfloat16)
    for name, ref in (("silu_mul", F.silu(aux) * y), ("mul_sigmoid", aux * torch.sigmoid(y))):
        got = ops.gate_op(y, aux, ops.EPILOGUES[name])
        torch.cuda.synchronize()
        assert got.shape == ref.shape and torch.equal(got, ref), f"{name} {shape}"


def test_gate_op_unaligned_views_and_in_place(dev):
    from krea2_svdquant_amd.kernels.hip import lib, ops
    gen = torch.Generator(device=dev).manual_seed(5)
    base = torch.randn(2, 1001, device=dev, generator=gen).to(torch.bfloat16)
    y, aux = base[0, 1:], base[1, :-1]                  # 2-byte offsets: copied to aligned buffers
    assert y.data_ptr() % 16 != 0
    got = ops.gate_op(y.contiguous(), aux.contiguous(), ops.EPILOGUES["silu_mul"])
    assert torch.equal(got, F.silu(aux) * y)
    # in place through the C-ABI: out == y
    y2 = (torch.randn(4099, device=dev, generator=gen) * 3).to(torch.bfloat16)
    a2 = (torch.randn(4099, device=dev, generator=gen) * 3).to(torch.bfloat16)
    ref = a2 * torch.sigmoid(y2)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    lib.call("svdq_gate_op", lib.SVDQ_EPI_MUL_SIGMOID, y2.data_ptr(), a2.data_ptr(), y2.data_ptr(), y2.numel(),
             stream)
    torch.cuda.synchronize()
    assert torch.equal(y2, ref)
