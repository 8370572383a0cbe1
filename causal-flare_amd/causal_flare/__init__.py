"""MI355X-native causal FLARE forward: a drop-in for the hot path of vpuri3/causal-flare.

Same public names as the reference package (``causal_flare/__init__.py:1-27``).
Every compute call runs hand-written HIP kernels for gfx950 from
``_lib/libflare_mi355x.so``; there is no CPU fallback.  Out of scope here and
raising ``NotImplementedError``: the semi-autoregressive prefill/decode stubs
(stubs in the reference too).
"""
from . import autoregressive, semi_autoregressive
from .autoregressive.training import flare_autoregressive_triton
from .autoregressive.recurrent import flare_recurrent_triton
from .autoregressive.inference import (
    flare_autoregressive_decode_triton,
    flare_autoregressive_prefill_triton,
)
from .semi_autoregressive.training import flare_semi_autoregressive_trition
from .semi_autoregressive.inference import (
    flare_semi_autoregressive_decode_trition,
    flare_semi_autoregressive_prefill_trition,
)

__version__ = "0.0.1+mi355x"


__all__ = [
    "autoregressive",
    "semi_autoregressive",
    "flare_autoregressive_triton",
    "flare_autoregressive_decode_triton",
    "flare_autoregressive_prefill_triton",
    "flare_recurrent_triton",
    "flare_semi_autoregressive_decode_trition",
    "flare_semi_autoregressive_prefill_trition",
    "flare_semi_autoregressive_trition",
    "__version__",
]
