"""MI355X (gfx950) SVDQuantLinear backend: hand-written HIP kernels behind the reference API.

Public names mirror the reference ``krea2_svdquant`` package where they exist there
(``BackendKind``, ``SVDQuantConfig``, ``SVDQuantLinearState``, ``SVDQuantLinear``,
``SVDQuantLoRAAdapter``) and add the backend function ``svdquant_linear_hip_gfx950``.
"""
from .config import BACKEND_CHOICES, BackendKind, SVDQuantConfig
from .quant.state import SVDQuantLinearState

__all__ = ["BACKEND_CHOICES", "BackendKind", "SVDQuantConfig", "SVDQuantLinearState",
           "SVDQuantLinear", "SVDQuantLoRAAdapter", "svdquant_linear_hip_gfx950",
           "svdquant_linear_hip_gfx950_w4a16"]


def __getattr__(name):
    if name in ("SVDQuantLinear", "SVDQuantLoRAAdapter"):
        from .runtime import linear
        return getattr(linear, name)
    if name in ("svdquant_linear_hip_gfx950", "svdquant_linear_hip_gfx950_w4a16"):
        from .kernels.hip import backend
        return getattr(backend, name)
    raise AttributeError(name)
