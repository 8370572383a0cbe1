from .training import AutoRegressiveFLARE, flare_autoregressive_triton
from .inference import flare_autoregressive_decode_triton, flare_autoregressive_prefill_triton

__all__ = [
    "AutoRegressiveFLARE",
    "flare_autoregressive_triton",
    "flare_autoregressive_decode_triton",
    "flare_autoregressive_prefill_triton",
]
