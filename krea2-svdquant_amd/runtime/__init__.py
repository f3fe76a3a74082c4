from .linear import SVDQuantLinear, SVDQuantLoRAAdapter

__all__ = ["SVDQuantLinear", "SVDQuantLoRAAdapter"]
