"""Host-side behaviour of the drop-in boundary (no GPU needed): the mirrored reference API, its
error behaviour, LoRA bookkeeping, the converter's agreement with the oracle, and loud failure
instead of any fallback."""
import numpy as np
import pytest
import torch

from krea2_svdquant_amd import BACKEND_CHOICES, BackendKind, SVDQuantConfig, SVDQuantLinearState
from krea2_svdquant_amd.quant import convert
from krea2_svdquant_amd.runtime.linear import SVDQuantLinear, SVDQuantLoRAAdapter
from oracle import numerics as nm
from oracle import pack as op


def _state(n=3, k=4, packed=True):
    return SVDQuantLinearState(
        smooth_scale=torch.ones(k, dtype=torch.bfloat16),
        qweight=torch.full((n, k // 2), 0x88, dtype=torch.uint8) if packed else torch.zeros(n, k, dtype=torch.int8),
        weight_scales=torch.ones(n, 1, dtype=torch.float16), l1=torch.zeros(n, 1, dtype=torch.bfloat16),
        l2=torch.zeros(1, k, dtype=torch.bfloat16), bias=None, group_size=k, original_shape=(n, k),
        qweight_packed=packed, padded_in_features=k if packed else None)


def test_backend_kind_keeps_reference_members_and_adds_hip():
    for v in ("auto", "pytorch_sim", "triton_generic", "triton_blackwell", "gluon_blackwell"):
        assert BackendKind(v).value == v
    assert BackendKind("hip_gfx950") is BackendKind.HIP_GFX950
    assert "hip_gfx950_w4a16" in BACKEND_CHOICES
    cfg = SVDQuantConfig()
    assert cfg.weight_group_size == 128 and cfg.rank_for("transformer_blocks.0.ff.up") == 64
    assert cfg.rank_for("transformer_blocks.0.attn.to_q") == 32


def test_module_buffers_state_and_lora_validation():
    mod = SVDQuantLinear(_state(), backend="hip_gfx950")
    names = {n for n, _ in mod.named_buffers()}
    assert {"smooth_scale", "qweight", "weight_scales", "l1", "l2"} <= names
    st = mod.state
    assert st.qweight_packed and st.original_shape == (3, 4) and st.group_size == 4
    with pytest.raises(ValueError, match="down input mismatch"):
        mod.add_lora_adapter(torch.zeros(2, 5), torch.zeros(3, 2))
    with pytest.raises(ValueError, match="up output mismatch"):
        mod.add_lora_adapter(torch.zeros(2, 4), torch.zeros(4, 2))
    with pytest.raises(ValueError, match="shape mismatch"):
        mod.add_lora_adapter(torch.zeros(2, 4), torch.zeros(3, 3))
    mod.add_lora_adapter(torch.zeros(2, 4), torch.zeros(3, 2), scale=0.5, network_alpha=4.0)
    assert len(mod.lora_adapters) == 1 and mod.lora_adapters[0].multiplier == 1.0
    assert SVDQuantLoRAAdapter(torch.zeros(8, 4), torch.zeros(3, 8), scale=0.8).multiplier == pytest.approx(0.8)


def test_forward_fails_loudly_without_gpu_or_hip_backend():
    x = torch.randn(2, 4).to(torch.bfloat16)
    with pytest.raises(RuntimeError):
        SVDQuantLinear(_state(), backend="hip_gfx950")(x)
    with pytest.raises(NotImplementedError, match="pytorch_sim"):
        SVDQuantLinear(_state(), backend="pytorch_sim")(x)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="gfx950"):
            SVDQuantLinear(_state(), backend="auto")(x)


def test_unpacked_state_rejected():
    from krea2_svdquant_amd.kernels.hip.backend import prepare_layer
    with pytest.raises(RuntimeError, match="packed"):
        prepare_layer(_state(packed=False), device="cpu")


def test_converter_matches_oracle_quantizer_bit_exact():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((48, 320)).astype(np.float32) * 0.02
    q_t, s_t = convert.quantize_symmetric_int4(torch.from_numpy(w), 64, dim=1)
    q_o, s_o = op.quantize_symmetric_int4(w, 64, "f32")
    assert np.array_equal(q_t.numpy(), q_o) and np.array_equal(s_t.numpy(), s_o)
    packed = convert.pack_int4(q_t)
    assert np.array_equal(packed.numpy(), op.pack_int4(q_o))
    assert torch.equal(convert.unpack_int4(packed, 320), q_t)
    xb = torch.from_numpy(rng.standard_normal((9, 130)).astype(np.float32)).to(torch.bfloat16)
    q_b, s_b = convert.quantize_symmetric_int4(xb, 64)
    q_ob, s_ob = op.quantize_symmetric_int4(xb.float().numpy(), 64, "bf16")
    assert np.array_equal(q_b.numpy(), q_ob) and np.array_equal(s_b.float().numpy(), s_ob)


def test_convert_linear_layout_and_reconstruction():
    torch.manual_seed(0)
    w = torch.randn(96, 256) * 0.02
    xs = torch.randn(64, 256)
    st = convert.convert_linear(w, torch.randn(96), xs.abs().amax(0), rank=8, group_size=64,
                                smooth_clamp=(None, None), seed=3)
    assert st.qweight.dtype == torch.uint8 and tuple(st.qweight.shape) == (96, 128)
    assert st.weight_scales.dtype == torch.float16 and tuple(st.weight_scales.shape) == (96, 4)
    assert st.smooth_scale.dtype == torch.bfloat16 and st.l1.dtype == torch.bfloat16
    assert st.qweight_packed and st.padded_in_features == 256 and st.bias.dtype == torch.bfloat16
    # W*s ~= dequant(residual) + L1 L2 to INT4 precision
    q = convert.unpack_int4(st.qweight, 256)
    res = convert.dequantize_symmetric_int4(q, st.weight_scales.float(), 64, dim=1)
    approx = res + st.l1.float() @ st.l2.float()
    target = w * st.smooth_scale.float()
    assert (approx - target).norm() / target.norm() < 0.1
    assert nm.bf16_bits(st.smooth_scale.float().numpy()).dtype == np.uint16


def test_epilogue_operand_validation_on_the_host():
    from krea2_svdquant_amd.kernels.hip import backend
    cpu = torch.device("cpu")
    aux = torch.zeros(4, 8, dtype=torch.bfloat16)
    assert backend._epilogue_operands("none", None, None, 4, 8, cpu) == (0, None, None)
    with pytest.raises(ValueError, match="epilogue must be one of"):
        backend._epilogue_operands("gelu", aux, None, 4, 8, cpu)
    with pytest.raises(ValueError, match="without an epilogue op"):
        backend._epilogue_operands("none", aux, None, 4, 8, cpu)
    with pytest.raises(ValueError, match="needs aux"):
        backend._epilogue_operands("silu_mul", aux[:, :4], None, 4, 8, cpu)
    with pytest.raises(TypeError, match="bfloat16"):
        backend._epilogue_operands("silu_mul", aux.float(), None, 4, 8, cpu)
    with pytest.raises(ValueError, match="needs vec"):
        backend._epilogue_operands("residual_gate", aux, None, 4, 8, cpu)
    with pytest.raises(ValueError, match="only used by"):
        backend._epilogue_operands("mul_sigmoid", aux, torch.zeros(8, dtype=torch.bfloat16), 4, 8, cpu)
    epi, a2, v2 = backend._epilogue_operands("residual_gate", aux.view(2, 2, 8), torch.ones(8), 4, 8, cpu)
    assert epi == 3 and tuple(a2.shape) == (4, 8) and v2.dtype == torch.bfloat16


def test_backend_function_caches_prepared_operands_per_state(monkeypatch):
    """The stateless backend function (the reference's ``fn(x, state)`` seam) prepares a state's
    kernel operands once and reuses them; an in-place edit of a buffer, a swapped buffer, a changed
    adapter multiplier or a new adapter set prepares again; the entry goes with its state."""
    import gc
    import types
    from krea2_svdquant_amd.kernels.hip import backend
    prepared = []
    monkeypatch.setattr(backend, "prepare_layer", lambda state, adapters, device: prepared.append(len(adapters)) or
                        object())
    monkeypatch.setattr(backend, "forward_prepared", lambda x, prep, **kw: prep)
    st = _state(n=8, k=64)
    x = torch.zeros(2, 64)
    a = backend.svdquant_linear_hip_gfx950(x, st)
    assert backend.svdquant_linear_hip_gfx950(x, st) is a and len(prepared) == 1
    st.l1.add_(1.0)                                      # in-place edit: version counter moves
    b = backend.svdquant_linear_hip_gfx950(x, st)
    assert b is not a and len(prepared) == 2
    st.bias = torch.zeros(8, dtype=torch.bfloat16)       # a new buffer
    backend.svdquant_linear_hip_gfx950(x, st)
    assert len(prepared) == 3
    ad = types.SimpleNamespace(down_weight=torch.zeros(4, 64), up_weight=torch.zeros(8, 4), multiplier=0.5)
    c = backend.svdquant_linear_hip_gfx950(x, st, adapters=[ad])
    assert backend.svdquant_linear_hip_gfx950(x, st, adapters=[ad]) is c and prepared[-1] == 1
    ad.multiplier = 0.25
    assert backend.svdquant_linear_hip_gfx950(x, st, adapters=[ad]) is not c
    key = id(st)
    assert key in backend._SEAM_CACHE
    del st
    gc.collect()
    assert key not in backend._SEAM_CACHE
