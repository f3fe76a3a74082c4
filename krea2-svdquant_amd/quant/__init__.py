from .state import SVDQuantLinearState
from .convert import (compute_smooth_scale, dequantize_symmetric_int4, pack_int4,
                      quantize_linear_from_samples, quantize_symmetric_int4, svd_lowrank, unpack_int4)

__all__ = [
    "SVDQuantLinearState", "compute_smooth_scale", "dequantize_symmetric_int4", "pack_int4",
    "quantize_linear_from_samples", "quantize_symmetric_int4", "svd_lowrank", "unpack_int4",
]
