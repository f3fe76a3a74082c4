"""Backend selection and quantization defaults (mirror of reference ``src/krea2_svdquant/config.py``).

``BackendKind`` keeps every reference member (``config.py:7-12``) so that a ``--backend``
string valid for the reference parses here too, and adds the two gfx950 backends of this
package:

* ``hip_gfx950``       -- W4A4: smoothing + dynamic per-group INT4 activations, and a GEMM of
  exact INT4-code group sums on the FP6 MFMA (every INT4 code is an e3m2 value; FP8 and INT8
  operand kernels stay selectable) with the low-rank / LoRA / bias epilogue fused (the path the
  reference plans in ``README.md:188-195``);
* ``hip_gfx950_w4a16`` -- W4A16: bf16 activations, INT4 weights dequantized in registers,
  BF16-MFMA GEMM; numerically the reference ``pytorch_sim`` math.

``AUTO`` resolves to ``hip_gfx950`` on a gfx950 device.  The Triton, Gluon and simulation
backends of the reference are not part of this package: selecting them raises.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum


class BackendKind(str, Enum):
    AUTO = "auto"
    PYTORCH_SIM = "pytorch_sim"
    TRITON_GENERIC = "triton_generic"
    TRITON_BLACKWELL = "triton_blackwell"
    GLUON_BLACKWELL = "gluon_blackwell"
    HIP_GFX950 = "hip_gfx950"
    HIP_GFX950_W4A16 = "hip_gfx950_w4a16"


BACKEND_CHOICES = tuple(b.value for b in BackendKind)
"""Values for a ``--backend`` argparse option (reference ``scripts/infer_svdquant_transformer.py:34-39``)."""


@dataclass(slots=True)
class SVDQuantConfig:
    """Quantization defaults, as in reference ``config.py:15-49`` (group 128, ranks 32/64)."""
    weight_bits: int = 4
    activation_bits: int = 4
    weight_group_size: int = 128
    activation_group_size: int = 128
    default_rank: int = 32
    mlp_rank: int = 64
    attn_rank: int = 32
    smooth_min: float = 0.25
    smooth_max: float = 4.0
    svd_oversample: int = 8
    svd_niter: int = 4
    lowrank_dtype: str = "bfloat16"
    output_dtype: str = "bfloat16"
    target_modules: tuple[str, ...] = field(
        default_factory=lambda: (
            "attn.to_q", "attn.to_k", "attn.to_v", "attn.to_gate", "attn.to_out.0",
            "ff.gate", "ff.up", "ff.down",
        )
    )

    def rank_for(self, module_name: str) -> int:
        if ".ff." in module_name or module_name.endswith(("ff.gate", "ff.up", "ff.down")):
            return self.mlp_rank
        if ".attn." in module_name or ".to_" in module_name:
            return self.attn_rank
        return self.default_rank
