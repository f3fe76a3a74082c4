"""GPU tests of the W4A16 GEMM on specialized waves (``w4a16_ws_kernel``) against the register-staged
kernel (``w4a16_wide_kernel``) on the same 192-row tiles.

Both compute each output the same way: weights dequantized to bf16(q * bf16(sw)), the same bf16
MFMAs over the same 16-column k-steps in the same order, then the low-rank term as hi_k then lo_k
slices of the mid planes against l1cat (in the epilogue there, as extra k-steps here), then bias and
the store.  So on every shape the outputs must be bit-identical.  ``SVDQ_W4A16_KERNEL=wide`` forces
the register-staged kernel; by default the specialized one takes the shapes whose 192-row tiles
need fewer rounds over the CUs than 256-row tiles (e.g. config 2's ff.up, M = 2304, N = 16384).
Parity of the default path against the oracle at config 2's shapes: ``test_gpu_config2_shapes.py``
and ``test_gpu_kernels.py::test_w4a16_wide_tiles``.
"""
import os
from contextlib import contextmanager

import pytest
import torch

pytestmark = pytest.mark.gpu


@contextmanager
def _kernel(name):
    old = os.environ.get("SVDQ_W4A16_KERNEL")
    if name is None:
        os.environ.pop("SVDQ_W4A16_KERNEL", None)
    else:
        os.environ["SVDQ_W4A16_KERNEL"] = name
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("SVDQ_W4A16_KERNEL", None)
        else:
            os.environ["SVDQ_W4A16_KERNEL"] = old


def _prepared(dev, n, k, group, seed, lora_ranks=()):
    from krea2_svdquant_amd.runtime.krea2_standin import random_quantized_state
    from krea2_svdquant_amd.runtime.linear import SVDQuantLinear
    gen = torch.Generator(device=dev).manual_seed(seed)
    st = random_quantized_state(n, k, rank=32, group_size=group, device=dev, generator=gen)
    st.bias = (torch.randn(n, device=dev, generator=gen) * 0.1).to(torch.bfloat16)
    mod = SVDQuantLinear(st, backend="hip_gfx950_w4a16")
    for r in lora_ranks:
        mod.add_lora_adapter((torch.randn(r, k, device=dev, generator=gen) * 0.02).to(torch.bfloat16),
                             (torch.randn(n, r, device=dev, generator=gen) * 0.02).to(torch.bfloat16), scale=0.8)
    return mod._prepare(dev, with_adapters=bool(lora_ranks))


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("m,n,k,group,lora", [
    (2304, 4096, 512, 64, ()),         # 192 tiles of 192 x 256, 8 stages + 1 low-rank stage
    (2100, 4300, 576, 64, ()),         # partial last tiles in M and N; 9 stages (odd)
    (2048, 4352, 640, 128, ()),        # group 128: 10 stages
    (2304, 16384, 384, 64, ()),        # config 2 ff.up's tiling at short K: 768 tiles
    (2304, 4096, 1024, 64, (48,)),     # LoRA: rank tiles of 96, three low-rank stages
    (1920, 4096, 256, 128, (64, 32)),  # LoRA rank 128 (four low-rank stages), 4 stages
])
def test_ws_kernel_bit_identical_to_register_staged(dev, m, n, k, group, lora, out_f32):
    from krea2_svdquant_amd.kernels.hip.backend import forward_prepared
    print(f"w4a16 ws vs wide: M={m} N={n} K={k} G={group} lora={lora} f32={out_f32}", flush=True)
    prep = _prepared(dev, n, k, group, seed=m + n + k + group, lora_ranks=lora)
    gen = torch.Generator(device=dev).manual_seed(5)
    x = (torch.randn(m, k, device=dev, generator=gen) * 2).to(torch.bfloat16)
    x[:, ::89] *= 20   # outlier channels
    with _kernel(None):
        a = forward_prepared(x, prep, mode="w4a16", out_f32=out_f32)
    with _kernel("wide"):
        b = forward_prepared(x, prep, mode="w4a16", out_f32=out_f32)
    torch.cuda.synchronize()
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)
