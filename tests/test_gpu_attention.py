"""GPU parity of the stand-in block's attention kernel (`svdq::attention`, `csrc/svdq_attn.hip`).

The reference is the float32 evaluation of softmax(scale q k^T) v on the same bf16 inputs,
per head with contiguous operands.  The kernel rounds the probabilities to bf16 before the
product with v (as PyTorch's fused SDPA kernels do) and the output to bf16 once, so it is held
to a relative L2 error of 4e-3 and, beside that, to an error no larger than twice SDPA's own on
the same inputs (SDPA flash / memory-efficient, the path the stand-in used before).
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _reference(q, k, v, scale):
    """float32 attention, one head at a time (q [T, H, d], k / v [T, Hkv, d]) -> [T, H, d]."""
    t, heads, d = q.shape
    g = heads // k.shape[1]
    out = torch.empty((t, heads, d), dtype=torch.float32, device=q.device)
    for hh in range(heads):
        qh = q[:, hh].float().contiguous()
        kh = k[:, hh // g].float().t().contiguous()
        vh = v[:, hh // g].float().contiguous()
        p = torch.softmax((qh @ kh) * scale, dim=-1)
        out[:, hh] = p @ vh
    return out


def _sdpa(q, k, v):
    from torch.nn.attention import SDPBackend, sdpa_kernel
    qh, kh, vh = (z.transpose(0, 1).unsqueeze(0).contiguous() for z in (q, k, v))
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        o = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, enable_gqa=True)
    return o.squeeze(0).transpose(0, 1)


def _rel(a, ref):
    return float((a.float() - ref).norm() / ref.norm())


def _check(q, k, v, tol=4e-3):
    from krea2_svdquant_amd.kernels.hip import ops
    scale = 1.0 / math.sqrt(q.shape[-1])
    out = ops.attention(q, k, v, scale)
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    ref = _reference(q, k, v, scale)
    err = _rel(out, ref)
    err_sdpa = _rel(_sdpa(q, k, v), ref)
    assert err <= tol, f"rel-L2 {err:.2e} against the float32 evaluation"
    assert err <= 2.0 * err_sdpa + 1e-4, f"rel-L2 {err:.2e}, SDPA {err_sdpa:.2e}"
    return out


def _inputs(t, heads, kvh, dev, seed, qscale=1.0):
    gen = torch.Generator(device=dev).manual_seed(seed)
    q = (torch.randn(t, heads, 128, device=dev, generator=gen) * qscale).to(torch.bfloat16)
    k = torch.randn(t, kvh, 128, device=dev, generator=gen).to(torch.bfloat16)
    v = torch.randn(t, kvh, 128, device=dev, generator=gen).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("t,heads,kvh", [
    (1, 4, 1),        # one key: softmax of a single score
    (7, 8, 2),        # one partial key tile, one partial query block
    (64, 8, 8),       # exactly one key tile, no grouping
    (65, 8, 2),       # a second tile holding one key
    (130, 12, 3),     # partial last tiles in both directions
    (300, 48, 12),    # the stand-in's head counts
])
def test_attention_matches_float32(dev, t, heads, kvh):
    q, k, v = _inputs(t, heads, kvh, dev, seed=t + heads)
    _check(q, k, v)


def test_attention_sharp_and_rising_scores(dev):
    """Large scores (a near one-hot softmax) whose maximum grows from key tile to key tile: every
    tile rescales the running output."""
    t, heads, kvh = 333, 8, 2
    q, k, v = _inputs(t, heads, kvh, dev, seed=5, qscale=6.0)
    ramp = torch.linspace(0.5, 3.0, t, device=dev).view(t, 1, 1)
    k = (k.float() * ramp).to(torch.bfloat16)
    _check(q, k, v, tol=6e-3)


def _fast_flags(q, k, v, scale):
    """Run the C-ABI entry point with a workspace of our own and return (output, the per-wave
    flags it leaves at the workspace's start: [H, 4 ceil(T / 256)] int32, 1 = query block
    written by the running-maximum kernel)."""
    import ctypes
    from krea2_svdquant_amd.kernels.hip import lib
    t, heads, kvh = q.shape[0], q.shape[1], k.shape[1]
    out = torch.empty_like(q)
    ws = torch.empty(lib.load().svdq_attention_workspace(t, heads), dtype=torch.uint8, device=q.device)
    vp = lambda z: ctypes.c_void_p(z.data_ptr())
    lib.call("svdq_attention_fwd", vp(q), q.stride(0), vp(k), vp(v), k.stride(0), t, heads, kvh,
             ctypes.c_float(scale), vp(out), out.stride(0), vp(ws),
             ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream))
    nflag = 4 * ((t + 255) // 256)
    flags = ws[: heads * nflag * 4].view(torch.int32).view(heads, nflag)
    return out, flags


def test_attention_scores_far_above_the_first_keys(dev):
    """Keys 0..31 near zero, every later key aligned with q: later scores sit ~65 (log2 units)
    above the first 32 keys' maximum (the fast kernel's fixed exponent offset), so the fast
    kernel's row sums pass 2^64 and its waves hand their queries to the running-maximum kernel,
    whose output is checked here."""
    t, heads, kvh = 200, 4, 2
    gen = torch.Generator(device=dev).manual_seed(13)
    q = (2.0 + 0.05 * torch.randn(t, heads, 128, device=dev, generator=gen)).to(torch.bfloat16)
    k = 2.0 + 0.05 * torch.randn(t, kvh, 128, device=dev, generator=gen)
    k[:32] = 0.01 * torch.randn(32, kvh, 128, device=dev, generator=gen)
    k = k.to(torch.bfloat16)
    v = torch.randn(t, kvh, 128, device=dev, generator=gen).to(torch.bfloat16)
    scores = (q[:1, 0].float() @ k[:, 0].float().t().contiguous()) / math.sqrt(128) * math.log2(math.e)
    assert float(scores[0, 32:].max() - scores[0, :32].max()) > 64
    out = _check(q, k, v)
    out2, flags = _fast_flags(q, k, v, 1.0 / math.sqrt(128))
    live = flags[:, : (t + 63) // 64]           # query blocks of 64 that hold queries below T
    assert bool((live == 1).all()), flags
    assert torch.equal(out2, out)


def test_attention_tail_pieces_hand_over_overflowing_products(dev):
    """T=300 at 48 query heads: 96 items, all in the last, partly filled round, so every item runs
    as key pieces merged by the combine kernel.  Keys 32.. score 56 log2 units above the first 32
    keys (the fixed exponent offset), so a probability reaches 2^56 while the row sum stays below
    2^64, and every v is 2^73: p v passes the f32 range in the first piece.  Those waves must hand
    their queries to the running-maximum kernel (as whole items do through their normalized
    output), and the output is the average of equal values, 2^73, exactly."""
    t, heads, kvh = 300, 48, 12
    q = torch.ones(t, heads, 128, device=dev, dtype=torch.bfloat16)
    s56 = 56.0 * math.log(2.0) * math.sqrt(128) / 128   # per-element k: q . k / sqrt(128) = 56 ln 2
    k = torch.full((t, kvh, 128), s56, device=dev)
    k[:32] = 0.0
    k = k.to(torch.bfloat16)
    v = torch.full((t, kvh, 128), 2.0 ** 73, device=dev, dtype=torch.bfloat16)
    out, flags = _fast_flags(q, k, v, 1.0 / math.sqrt(128))
    live = flags[:, : (t + 63) // 64]
    assert bool((live == 1).all()), flags
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out, torch.full_like(out, 2.0 ** 73))


def test_attention_random_inputs_stay_on_the_fast_kernel(dev):
    """N(0, 1) inputs at the config-3 head counts: no fast wave hands its queries over."""
    q, k, v = _inputs(1000, 48, 12, dev, seed=21)
    _, flags = _fast_flags(q, k, v, 1.0 / math.sqrt(128))
    assert int(flags.sum()) == 0


def test_attention_strided_rows(dev):
    """q, k, v as head slices of wider rows (row strides above the heads' width)."""
    t, heads, kvh = 200, 8, 2
    gen = torch.Generator(device=dev).manual_seed(9)
    fused = torch.randn(t, (heads + 2 * kvh + 1) * 128, device=dev, generator=gen).to(torch.bfloat16)
    q = fused[:, : heads * 128].view(t, heads, 128)
    k = fused[:, heads * 128: (heads + kvh) * 128].view(t, kvh, 128)
    v = fused[:, (heads + kvh) * 128: (heads + 2 * kvh) * 128].view(t, kvh, 128)
    assert q.stride(0) == fused.shape[1] and not q.is_contiguous()
    _check(q, k, v)


def test_attention_config3_shape(dev):
    """The stand-in block at config 3: 4096 latent + 256 text tokens, 48 query heads over 12."""
    q, k, v = _inputs(4352, 48, 12, dev, seed=3)
    _check(q, k, v)


def test_attention_rejects_bad_shapes(dev):
    from krea2_svdquant_amd.kernels.hip import ops
    q, k, v = _inputs(16, 6, 4, dev, seed=1)
    with pytest.raises(ValueError):
        ops.attention(q, k, v, 0.1)                     # 6 heads over 4
    with pytest.raises(ValueError):
        ops.attention(q[..., :64].contiguous(), k, v, 0.1)
    q2, k2, v2 = _inputs(16, 8, 2, dev, seed=2)
    with pytest.raises(ValueError):
        ops.attention(q2, k2, v2[:8], 0.1)


@pytest.mark.parametrize("t,heads,kvh,kscale", [(300, 4, 2, 1.0), (4352, 48, 12, 1.0), (200, 4, 2, 25.0)])
def test_attention_qnorm_matches_head_norm_then_attention(dev, t, heads, kvh, kscale):
    """svdq::attention_qnorm (q's per-head norm + rotary applied on load) against
    svdq::head_rms_rope followed by svdq::attention: the normalized q may differ by one bf16 ulp
    where the mean of squares sits at a rounding boundary, so the outputs agree to rel-L2 1e-3;
    both against the float32 evaluation on the normalized q.  kscale 25 drives rows past the fast
    kernel's offset limit (the running-maximum kernel normalizes q as well)."""
    from krea2_svdquant_amd.kernels.hip import ops
    from krea2_svdquant_amd.runtime.krea2_standin import rope_tables
    gen = torch.Generator(device=dev).manual_seed(t + heads)
    q = (torch.randn(t, heads, 128, device=dev, generator=gen) * 3).to(torch.bfloat16)
    k = (torch.randn(t, kvh, 128, device=dev, generator=gen) * kscale).to(torch.bfloat16)
    v = torch.randn(t, kvh, 128, device=dev, generator=gen).to(torch.bfloat16)
    cos, sin = rope_tables(t, 128, dev, torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    qn = ops.head_rms_rope(q, cos, sin, 1e-6)
    ref_path = ops.attention(qn, k, v, scale)
    got = ops.attention_qnorm(q, k, v, cos, sin, 1e-6, scale)
    torch.cuda.synchronize()
    assert got.shape == q.shape and got.dtype == torch.bfloat16
    assert _rel(got, ref_path.float()) <= 1e-3
    ref = _reference(qn, k, v, scale)
    assert _rel(got, ref) <= 4e-3 and _rel(ref_path, ref) <= 4e-3
