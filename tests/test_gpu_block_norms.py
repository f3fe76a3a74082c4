"""GPU tests of the stand-in block's normalization kernels (``svdq::rms_norm_modulate``,
``svdq::head_rms_rope``) against the torch ops the block runs on the CPU:

* ``F.rms_norm(x, weight=1 + scale) + shift``;
* ``apply_rope(F.rms_norm(t), cos, sin)`` per head of 128.

Both round where those ops round; the float32 mean of squares is summed in another order, so a
normalized value may move by one bf16 ulp where its float value sits at a rounding boundary, and
the shift or the rotary's difference of products carries that ulp into the output.  Bound: one
ulp of the normalized value plus one of the output, everywhere; bit-equal almost everywhere.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ulp(t: torch.Tensor) -> torch.Tensor:
    _, e = torch.frexp(t.float())
    return torch.ldexp(torch.ones_like(t, dtype=torch.float32), torch.clamp(e - 8, min=-133))


def _check(got, ref, norm, what):
    """got within ulp(norm) + ulp(ref) of ref (norm: the normalized values feeding each output)."""
    assert got.dtype == torch.bfloat16 and got.shape == ref.shape
    diff = (got.float() - ref.float()).abs()
    bound = _ulp(norm) + _ulp(ref)
    assert bool((diff <= bound).all()), f"{what}: max diff / bound {float((diff / bound).max())}"
    same = float((got == ref).float().mean())
    print(f"  {what}: bit-equal {same:.5f}")
    assert same > 0.99, f"{what}: only {same:.4f} bit-equal"


@pytest.mark.parametrize("t,h,ld", [(4352, 6144, 6144), (257, 1024, 1024), (33, 6144, 6160), (5, 8200, 8200)])
def test_rms_norm_modulate_matches_torch(dev, t, h, ld):
    """Rows held in registers between the passes (H <= 8192) and re-read (H = 8200); a leading
    dimension beyond H."""
    from krea2_svdquant_amd.kernels.hip import ops
    from krea2_svdquant_amd.runtime.krea2_standin import rms_norm
    gen = torch.Generator(device=dev).manual_seed(t + h)
    big = (torch.randn(t, ld, device=dev, generator=gen) * 3).to(torch.bfloat16)
    x = big[:, :h]
    scale = (torch.randn(h, device=dev, generator=gen) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(h, device=dev, generator=gen) * 0.1).to(torch.bfloat16)
    w = 1 + scale
    got = ops.rms_norm_modulate(x, w, shift, 1e-6)
    norm = rms_norm(x, 1e-6, weight=w)
    ref = norm + shift
    torch.cuda.synchronize()
    _check(got, ref, norm, f"rms_norm_modulate T={t} H={h}")


@pytest.mark.parametrize("t,heads,aligned", [(4352, 48, True), (4352, 12, True), (77, 3, True), (1, 1, True),
                                             (77, 3, False)])
def test_head_rms_rope_matches_torch(dev, t, heads, aligned):
    """16-byte kernel for aligned rows (the stand-in's case); the element-wise kernel for a view at
    an odd element offset."""
    from krea2_svdquant_amd.kernels.hip import ops
    from krea2_svdquant_amd.runtime.krea2_standin import apply_rope, rms_norm, rope_tables
    gen = torch.Generator(device=dev).manual_seed(t * heads)
    src = (torch.randn(t * heads * 128 + 1, device=dev, generator=gen) * 2).to(torch.bfloat16)
    q = (src[:-1] if aligned else src[1:]).view(t, heads, 128)
    assert (q.data_ptr() % 16 == 0) == aligned
    cos, sin = rope_tables(t, 128, dev, torch.bfloat16)
    got = ops.head_rms_rope(q, cos, sin, 1e-6)
    norm = rms_norm(q, 1e-6)
    ref = apply_rope(norm, cos, sin)
    # each output mixes the pair (j, j + 64): bound by the larger normalized value of the pair
    pair = torch.maximum(norm[..., :64].float().abs(), norm[..., 64:].float().abs())
    torch.cuda.synchronize()
    _check(got, ref, 2 * torch.cat([pair, pair], -1), f"head_rms_rope T={t} heads={heads}")


def test_block_norm_ops_reject_bad_shapes(dev):
    from krea2_svdquant_amd.kernels.hip import lib, ops
    x = torch.zeros(4, 12, device=dev, dtype=torch.bfloat16)
    v = torch.zeros(12, device=dev, dtype=torch.bfloat16)
    with pytest.raises(lib.SVDQError, match="H % 8"):
        ops.rms_norm_modulate(x, v, v, 1e-6)
    t = torch.zeros(4, 2, 64, device=dev, dtype=torch.bfloat16)
    tab = torch.zeros(4, 128, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="128"):
        ops.head_rms_rope(t, tab, tab, 1e-6)


@pytest.mark.parametrize("t,h,ld", [(4352, 6144, 6144), (257, 1024, 1024), (33, 6144, 6160), (5, 8200, 8200)])
def test_residual_rms_norm_modulate(dev, t, h, ld):
    """xo = the gated residual in one rounding, against torch.addcmul (one bf16 ulp of xo where
    torch's float product and sum round differently from one fused multiply-add; bit-equal almost
    everywhere), and y bit-equal to svdq::rms_norm_modulate of that xo: the residual changes
    nothing in the norm.  Rows in registers and re-read (H = 8200), a leading dimension beyond H."""
    from krea2_svdquant_amd.kernels.hip import ops
    gen = torch.Generator(device=dev).manual_seed(3 * t + h)
    big = (torch.randn(2, t, ld, device=dev, generator=gen) * 3).to(torch.bfloat16)
    x, v = big[0, :, :h], big[1, :, :h]
    gate = (torch.rand(h, device=dev, generator=gen) + 0.2).to(torch.bfloat16)
    w = (1 + torch.randn(h, device=dev, generator=gen) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(h, device=dev, generator=gen) * 0.1).to(torch.bfloat16)
    xo, y = ops.residual_rms_norm_modulate(x, v, gate, w, shift, 1e-6)
    ref = torch.addcmul(x, gate, v)
    torch.cuda.synchronize()
    diff = (xo.float() - ref.float()).abs()
    assert bool((diff <= _ulp(ref)).all()), "residual beyond one bf16 ulp of torch.addcmul"
    assert float((xo == ref).float().mean()) > 0.999
    assert torch.equal(y, ops.rms_norm_modulate(xo, w, shift, 1e-6))
