"""ctypes binding of ``libsvdq_gfx950.so`` (the C-ABI declared in ``include/svdq_gfx950.h``).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7`` dependency
resolves to the HIP runtime torch already loaded.  There is no fallback: if the library is
missing or fails to load, every entry raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the library load: HIP runtime binding)

PKG_DIR = Path(__file__).resolve().parents[2]
LIB_PATH = Path(os.environ.get("SVDQ_GFX950_LIB", PKG_DIR / "_lib" / "libsvdq_gfx950.so"))

SVDQ_ACT_PACKED = 1
SVDQ_ACT_XHAT = 2
SVDQ_ACT_EXACT_DIV = 4
SVDQ_ACT_OPERAND_E4M3 = 8
SVDQ_ACT_OPERAND_I8 = 16
SVDQ_ACT_SX_PAIRS = 32
SVDQ_ACT_OPERAND_E3M2 = 64

# split-partial floats of the device scratch of svdq_act_quant_noalloc (SVDQ_ACT_NOALLOC_MAX_FLOATS)
SVDQ_ACT_NOALLOC_MAX_FLOATS = 4 << 20

# epilogue ops of the *_gemm_epi entry points
SVDQ_EPI_NONE = 0
SVDQ_EPI_MUL_SIGMOID = 1
SVDQ_EPI_SILU_MUL = 2
SVDQ_EPI_RESIDUAL_GATE = 3

# sibling layers of one svdq_w4a4_gemm_siblings / svdq_w4a16_gemm_siblings call (SVDQ_MAX_SIBLINGS)
SVDQ_MAX_SIBLINGS = 4

STATUS = {0: "SVDQ_OK", -1: "SVDQ_ERR_ARG", -2: "SVDQ_ERR_SHAPE", -3: "SVDQ_ERR_ALIGN",
          -4: "SVDQ_ERR_UNSUPPORTED", -5: "SVDQ_ERR_LAUNCH"}

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_U = ctypes.c_uint


class ActSibling(ctypes.Structure):
    """``svdq_act_sibling``: one layer of ``svdq_act_quant_siblings``."""
    _fields_ = [("srs", _P), ("l2", _P), ("r", _I), ("qa", _P), ("sx", _P), ("mid", _P)]


class W4A4Sibling(ctypes.Structure):
    """``svdq_w4a4_sibling``: one layer of ``svdq_w4a4_gemm_siblings``."""
    _fields_ = [("qa", _P), ("sxp", _P), ("qwe", _P), ("swp", _P), ("mid", _P), ("l1cat", _P), ("RTp", _I),
                ("bias", _P), ("N", _I), ("y", _P), ("ldy", _L)]


class W4A16Sibling(ctypes.Structure):
    """``svdq_w4a16_sibling``: one layer of ``svdq_w4a16_gemm_siblings``."""
    _fields_ = [("xhat", _P), ("ldxh", _L), ("qw", _P), ("sw", _P), ("mid", _P), ("l1cat", _P), ("RTp", _I),
                ("bias", _P), ("N", _I), ("y", _P), ("ldy", _L)]


# name -> (restype, argtypes); the exact set of symbols include/svdq_gfx950.h declares.
SIGNATURES = {
    "svdq_version": (ctypes.c_char_p, []),
    "svdq_last_error": (ctypes.c_char_p, []),
    "svdq_group_supported": (_I, [_I]),
    "svdq_prepare_smooth": (_I, [_P, _P, _I, _P]),
    "svdq_act_quant_workspace": (_I, [_I, _I, _I, _I, ctypes.POINTER(_I), ctypes.POINTER(_L)]),
    "svdq_act_quant": (_I, [_P, _L, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _U, _P, _P, _P, _P, _L,
                            _P, _I, _P]),
    "svdq_act_quant_noalloc": (_I, [_P, _L, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _U, _P, _P, _P, _P, _L,
                                    _P, _P]),
    "svdq_prepare_weight_scales": (_I, [_P, _P, _I, _I, _I, _P]),
    "svdq_prepare_weight_operand": (_I, [_P, _P, _I, _I, _I, _P]),
    "svdq_w4a4_gemm": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _L, _I, _P]),
    "svdq_w4a16_gemm": (_I, [_P, _L, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _L, _I, _P]),
    "svdq_w4a4_gemm_tile_cols": (_I, [_I, _I, _I, _I, _I]),
    "svdq_w4a4_gemm_epi": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _L, _I,
                                _I, _P, _L, _P, _P]),
    "svdq_w4a16_gemm_epi": (_I, [_P, _L, _P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _L, _I,
                                 _I, _P, _L, _P, _P]),
    "svdq_act_quant_siblings": (_I, [_P, _L, ctypes.POINTER(ActSibling), _I, _I, _I, _I, _I, _U, _I, _P]),
    "svdq_w4a4_gemm_siblings": (_I, [ctypes.POINTER(W4A4Sibling), _I, _I, _I, _I, _I, _I, _P]),
    "svdq_w4a16_gemm_siblings": (_I, [ctypes.POINTER(W4A16Sibling), _I, _I, _I, _I, _I, _P]),
    "svdq_gate_op": (_I, [_I, _P, _P, _P, _L, _P]),
    "svdq_rms_norm_modulate": (_I, [_P, _L, _P, _P, _I, _I, ctypes.c_float, _P, _L, _P]),
    "svdq_residual_rms_norm_modulate": (_I, [_P, _L, _P, _L, _P, _P, _P, _I, _I, ctypes.c_float, _P, _L, _P, _L,
                                             _P]),
    "svdq_head_rms_rope": (_I, [_P, _I, _I, _P, _P, _L, ctypes.c_float, _P, _P]),
    "svdq_attention_workspace": (_L, [_I, _I]),
    "svdq_attention_fwd": (_I, [_P, _L, _P, _P, _L, _I, _I, _I, ctypes.c_float, _P, _L, _P, _P]),
    "svdq_attention_fwd_qnorm": (_I, [_P, _L, _P, _P, _L, _I, _I, _I, ctypes.c_float, _P, _P, _L, ctypes.c_float,
                                      _P, _L, _P, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class SVDQError(RuntimeError):
    """A C-ABI call returned a non-zero svdq_status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with {STATUS.get(status, status)}: {message}")
        self.status = status


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argument types set."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"gfx950 kernel library not found at {LIB_PATH}; build it with "
                    "__graft_entry__.build() (hipcc --offload-arch=gfx950)")
            lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise ``SVDQError`` on a non-zero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        raise SVDQError(name, status, lib.svdq_last_error().decode())


def version() -> str:
    return load().svdq_version().decode()


def w4a4_tile_cols(m: int, n: int, k: int, group: int, operand: int) -> int:
    """Columns of the block tile ``svdq_w4a4_gemm`` runs for this shape (256 or 128), 0 when the
    shape takes another kernel (``svdq_w4a4_gemm_tile_cols``)."""
    return int(load().svdq_w4a4_gemm_tile_cols(m, n, k, group, operand))
