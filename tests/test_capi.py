"""The C-ABI library: built, loadable, exports exactly what include/svdq_gfx950.h declares, and
validates arguments on the host (calls that fail validation make no GPU call)."""
import ctypes
import re
from pathlib import Path

import pytest

from krea2_svdquant_amd.kernels.hip import lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "svdq_gfx950.h"


def declared_symbols() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(svdq_[a-z0-9_]+)\s*\(", text))


def test_library_loads_and_exports_every_declared_symbol():
    handle = lib.load()
    decl = declared_symbols()
    assert decl == set(lib.SIGNATURES), "ctypes signatures out of sync with the header"
    for name in decl:
        assert getattr(handle, name) is not None
    assert lib.version().startswith("svdq_gfx950")


def test_group_support_and_workspace_sizing():
    h = lib.load()
    assert h.svdq_group_supported(64) == 1 and h.svdq_group_supported(128) == 1
    # any other multiple of 16 takes the generic kernels
    assert h.svdq_group_supported(32) == 1 and h.svdq_group_supported(16) == 1 and h.svdq_group_supported(192) == 1
    assert h.svdq_group_supported(24) == 0 and h.svdq_group_supported(0) == 0
    s, mp = ctypes.c_int(), ctypes.c_int64()
    lib.call("svdq_act_quant_workspace", 4096, 6144, 64, 32, ctypes.byref(s), ctypes.byref(mp))
    assert s.value >= 1 and mp.value == (s.value + 1) * 4096 * 32   # finalized head + one partial per split
    lib.call("svdq_act_quant_workspace", 256, 6144, 64, 32, ctypes.byref(s), ctypes.byref(mp))
    assert 1 < s.value <= 6144 // 64 // 4


@pytest.mark.parametrize("args,status,needle", [
    ((4096, 6144, 24, 32), -4, "group size 24"),
    ((4096, 6160, 16, 32), -2, "K % 64"),            # generic group sizes need K % 64 == 0
    ((4096, 6100, 64, 32), -2, "multiple of group"),
    ((4096, 6144, 64, 48), -2, "RTp=48"),
    ((0, 6144, 64, 32), -1, "M=0"),
])
def test_workspace_rejects_bad_arguments(args, status, needle):
    s, mp = ctypes.c_int(), ctypes.c_int64()
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_act_quant_workspace", *args, ctypes.byref(s), ctypes.byref(mp))
    assert ei.value.status == status and needle in str(ei.value)


def test_gemm_rejects_null_and_misaligned_pointers_before_any_launch():
    nul = None
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm", nul, 0, nul, nul, nul, nul, nul, 32, nul, 128, 128, 128, 64, nul, 128, 0, nul)
    assert ei.value.status == -1
    fake = ctypes.c_void_p(0x1000)
    odd = ctypes.c_void_p(0x1008)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm", fake, 0, fake, odd, fake, fake, fake, 32, nul, 128, 128, 128, 64, fake, 128, 0, nul)
    assert ei.value.status == -3
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a16_gemm", fake, 100, fake, fake, fake, fake, 32, nul, 128, 128, 128, 64, fake, 128, 0, nul)
    assert ei.value.status == -3
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_act_quant", fake, 128, fake, fake, 200, nul, 0, nul, 64, 128, 64, 192, lib.SVDQ_ACT_OPERAND_E4M3,
                 fake, fake, nul, nul, 0, fake, 1, nul)
    assert ei.value.status == -2 and "RTp=192" in str(ei.value)   # RTp < r + rl
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_act_quant", fake, 128, fake, fake, 32, nul, 0, nul, 64, 128, 64, 32,
                 lib.SVDQ_ACT_OPERAND_E4M3 | lib.SVDQ_ACT_OPERAND_I8, fake, fake, nul, nul, 0, fake, 1, nul)
    assert ei.value.status == -1 and "two operand formats" in str(ei.value)


def test_prepare_entry_points_reject_bad_arguments_before_any_launch():
    nul, fake = None, ctypes.c_void_p(0x1000)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_prepare_weight_operand", nul, fake, 128, 128, 0, nul)
    assert ei.value.status == -1
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_prepare_weight_operand", fake, fake, 128, 120, 0, nul)
    assert ei.value.status == -2 and "K % 16" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_prepare_weight_operand", fake, fake, 128, 128, 7, nul)
    assert ei.value.status == -1 and "operand format" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_prepare_weight_operand", fake, ctypes.c_void_p(0x1004), 128, 128, 0, nul)
    assert ei.value.status == -3
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_prepare_weight_scales", fake, fake, 0, 96, 0, nul)
    assert ei.value.status == -1


def test_w4a4_gemm_rejects_operands_beyond_32bit_offsets():
    fake = ctypes.c_void_p(0x1000)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm", fake, 0, fake, fake, fake, fake, fake, 32, None, 65536, 128, 65536, 64, fake, 128,
                 0, None)
    assert ei.value.status == -2 and "2^31" in str(ei.value)


@pytest.mark.parametrize("fn", ["svdq_w4a4_gemm_epi", "svdq_w4a16_gemm_epi"])
@pytest.mark.parametrize("epi,out_f32,aux,ldaux,vec,status,needle", [
    (7, 0, 0x1000, 128, None, -1, "epilogue op 7"),
    (lib.SVDQ_EPI_SILU_MUL, 1, 0x1000, 128, None, -1, "bf16 output"),
    (lib.SVDQ_EPI_MUL_SIGMOID, 0, None, 128, None, -1, "null epilogue operand"),
    (lib.SVDQ_EPI_RESIDUAL_GATE, 0, 0x1000, 128, None, -1, "null epilogue operand"),
    (lib.SVDQ_EPI_SILU_MUL, 0, 0x1000, 120, None, -2, "ldaux=120"),
    (lib.SVDQ_EPI_SILU_MUL, 0, 0x1001, 128, None, -3, "2-byte aligned"),
    (lib.SVDQ_EPI_RESIDUAL_GATE, 0, 0x1000, 136, 0x1003, -3, "2-byte aligned"),
])
def test_gemm_epilogue_ops_rejected_before_any_launch(fn, epi, out_f32, aux, ldaux, vec, status, needle):
    fake = ctypes.c_void_p(0x1000)
    aux_p = None if aux is None else ctypes.c_void_p(aux)
    vec_p = None if vec is None else ctypes.c_void_p(vec)
    if fn == "svdq_w4a4_gemm_epi":
        args = (fake, 2, fake, fake, fake, fake, fake, 32, None, 128, 128, 128, 64, fake, 128, out_f32)
    else:
        args = (fake, 128, fake, fake, fake, fake, 32, None, 128, 128, 128, 64, fake, 128, out_f32)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call(fn, *args, epi, aux_p, ldaux, vec_p, None)
    assert ei.value.status == status and needle in str(ei.value)



@pytest.mark.parametrize("m,k,g,rtp,status,needle", [
    (40000, 6144, 64, 128, -2, "device scratch"),   # 1 split x 40000 x 128 floats > 4 Mi floats
    (0, 6144, 64, 32, -1, "M=0"),
    (4096, 6144, 64, 40, -2, "RTp=40"),
    (4096, 6144, 40, 32, -4, "group size 40"),
])
def test_act_quant_noalloc_rejects_before_any_launch(m, k, g, rtp, status, needle):
    """The no-allocation entry point refuses a split-partial buffer beyond its device scratch
    (SVDQ_ACT_NOALLOC_MAX_FLOATS) and bad shapes on the host, before it touches the GPU."""
    fake = ctypes.c_void_p(0x1000)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_act_quant_noalloc", fake, k, fake, fake, 32, None, 0, None, m, k, g, rtp,
                 lib.SVDQ_ACT_OPERAND_E3M2 | lib.SVDQ_ACT_SX_PAIRS, fake, fake, None, None, k, fake, None)
    assert ei.value.status == status and needle in str(ei.value)
    splits = ctypes.c_int()
    if m > 0 and rtp % 32 == 0 and g == 64:
        lib.call("svdq_act_quant_workspace", m, k, g, rtp, ctypes.byref(splits), None)
        assert splits.value * m * rtp > lib.SVDQ_ACT_NOALLOC_MAX_FLOATS


def test_generic_group_rejects_fast_only_formats_before_any_launch():
    """Group sizes other than 64 / 128 run the generic kernels: int8 operands only, quantized from
    x_hat (the caller passes SVDQ_ACT_XHAT), and no fused epilogue ops."""
    fake, nul = ctypes.c_void_p(0x1000), None
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_act_quant", fake, 128, fake, fake, 32, nul, 0, nul, 64, 128, 32, 32,
                 lib.SVDQ_ACT_OPERAND_E3M2 | lib.SVDQ_ACT_SX_PAIRS, fake, fake, nul, nul, 0, fake, 1, nul)
    assert ei.value.status == -4 and "int8 operands only" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_act_quant", fake, 128, fake, fake, 32, nul, 0, nul, 64, 128, 32, 32,
                 lib.SVDQ_ACT_OPERAND_I8 | lib.SVDQ_ACT_SX_PAIRS, fake, fake, nul, nul, 0, fake, 1, nul)
    assert ei.value.status == -1 and "SVDQ_ACT_XHAT" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm", fake, 2, fake, fake, fake, fake, fake, 32, nul, 128, 128, 128, 32, fake, 128, 0, nul)
    assert ei.value.status == -4 and "int8 operands only" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm_epi", fake, 1, fake, fake, fake, fake, fake, 32, nul, 128, 128, 128, 32, fake, 128,
                 0, lib.SVDQ_EPI_SILU_MUL, fake, 128, nul, nul)
    assert ei.value.status == -4 and "epilogue" in str(ei.value)


def test_gate_op_and_siblings_reject_bad_arguments_before_any_launch():
    fake = ctypes.c_void_p(0x1000)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_gate_op", 3, fake, fake, fake, 8, None)
    assert ei.value.status == -1 and "op=3" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_gate_op", lib.SVDQ_EPI_SILU_MUL, ctypes.c_void_p(0x1002), fake, fake, 8, None)
    assert ei.value.status == -3
    lib.call("svdq_gate_op", lib.SVDQ_EPI_SILU_MUL, fake, fake, fake, 0, None)   # nothing to do
    layers = (lib.W4A4Sibling * 5)()
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm_siblings", layers, 5, 2, 256, 1024, 64, 0, None)
    assert ei.value.status == -1 and "count=5" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm_siblings", layers, 2, 2, 256, 1024, 64, 0, None)   # N = 0
    assert ei.value.status == -1 and "N=0" in str(ei.value)
    layers[0].N = layers[1].N = 128
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a4_gemm_siblings", layers, 2, 2, 256, 1024, 64, 0, None)   # null pointers
    assert ei.value.status == -1 and "null pointer" in str(ei.value)
    w16 = (lib.W4A16Sibling * 5)()
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a16_gemm_siblings", w16, 5, 256, 1024, 64, 0, None)
    assert ei.value.status == -1 and "count=5" in str(ei.value)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a16_gemm_siblings", w16, 2, 256, 1024, 64, 0, None)   # N = 0
    assert ei.value.status == -1 and "N=0" in str(ei.value)
    for lay in w16[:2]:
        lay.N, lay.RTp, lay.ldy, lay.ldxh = 128, 32, 128, 1024
        lay.qw = lay.sw = lay.mid = lay.l1cat = lay.y = 0x1000
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a16_gemm_siblings", w16, 2, 256, 1024, 64, 0, None)   # x_hat missing
    assert ei.value.status == -1 and "null xhat" in str(ei.value)
    w16[0].xhat = w16[1].xhat = 0x1008
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_w4a16_gemm_siblings", w16, 2, 256, 1024, 64, 0, None)   # x_hat not 16-byte aligned
    assert ei.value.status == -3 and "xhat" in str(ei.value)


def test_attention_qnorm_rejects_bad_tables_before_any_launch():
    fake = ctypes.c_void_p(0x1000)
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_attention_fwd_qnorm", fake, 1536, fake, fake, 1536, 16, 12, 12, ctypes.c_float(0.1), None,
                 fake, 64, ctypes.c_float(1e-6), fake, 1536, fake, None)
    assert ei.value.status == -1
    with pytest.raises(lib.SVDQError) as ei:
        lib.call("svdq_attention_fwd_qnorm", fake, 1536, fake, fake, 1536, 16, 12, 12, ctypes.c_float(0.1), fake,
                 fake, 60, ctypes.c_float(1e-6), fake, 1536, fake, None)
    assert ei.value.status == -3


def test_w4a4_tile_choice():
    """The host-side tiling rule: the 256 x 256 tiles where they need no more rounds of work per CU
    (at their measured 10% lower time per block), the 256 x 128 tiles elsewhere; 0 for shapes that
    take another kernel.  SVDQ_W4A4_TILES overrides (the wide tiles only where they apply)."""
    import os
    e3m2, i8 = 2, 1
    t = lib.w4a4_tile_cols
    assert t(4096, 16384, 6144, 64, e3m2) == 256      # config 1 ff.up: 4 rounds of 256 x 256, 8 of 256 x 128
    assert t(4096, 6144, 16384, 64, e3m2) == 128      # ff.down: 2 rounds x 2 against 3
    assert t(4096, 1536, 6144, 64, e3m2) == 128       # to_k: one round either way
    assert t(16384, 16384, 6144, 64, e3m2) == 256     # config 4 ff.up
    assert t(16384, 6144, 16384, 64, e3m2) == 256     # config 4 ff.down: 6 rounds x 2 x 0.9 < 12
    assert t(4352, 6144, 6144, 64, e3m2) == 256       # config 3 (4352 = 17 x 256)
    assert t(4000, 16384, 6144, 64, e3m2) == 128      # M not a multiple of 256
    assert t(4096, 16384, 6144, 128, e3m2) == 128     # group 128
    assert t(4096, 16384, 6144, 64, i8) == 0 and t(4096, 16384, 6144, 32, e3m2) == 0
    old = os.environ.get("SVDQ_W4A4_TILES")
    try:
        os.environ["SVDQ_W4A4_TILES"] = "256x128"
        assert t(4096, 16384, 6144, 64, e3m2) == 128
        os.environ["SVDQ_W4A4_TILES"] = "256x256"
        assert t(256, 256, 256, 64, e3m2) == 256 and t(300, 256, 256, 64, e3m2) == 128
    finally:
        if old is None:
            os.environ.pop("SVDQ_W4A4_TILES", None)
        else:
            os.environ["SVDQ_W4A4_TILES"] = old
