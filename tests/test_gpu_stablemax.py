"""GPU parity of the stablemax variant (flare_autoregressive_stablemax_triton,
C flare_stablemax_forward) against the fp64 oracle ``brute_stablemax``, which
tests/test_oracle.py pins to the chunked form of the reference's PyTorch path
(stablemax.py:578-635) and to closed forms.  Tolerances: tests/_util.py."""
import sys

import numpy as np
import pytest
import torch

import flare_oracle as O
from _util import assert_parity, seeded

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(*args):
    print("CASE", *args, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("power", [1.0, 2.0, 3.0, 4.0, 2.5])
def test_stablemax_forward(dtype, power):
    from causal_flare.autoregressive import flare_autoregressive_stablemax_triton
    _case("stablemax", dtype, power)
    B, N, H, M, D = 2, 203, 2, 64, 32
    q, k, v = seeded(70, B, N, H, M, D, D, dtype, q_std=D ** -0.5)
    ref = O.brute_stablemax(q, k, v, power=power)
    for chunk in (None, 16, 48):
        y = flare_autoregressive_stablemax_triton(q.to(DEV), k.to(DEV), v.to(DEV), power=power, chunk_size=chunk)
        assert y.dtype == dtype
        assert_parity(y, ref, dtype, f"stablemax power={power} chunk={chunk}")


@pytest.mark.parametrize("mode", ["sep_q", "sep_k", "both"])
def test_stablemax_separate_decoder(mode):
    from causal_flare.autoregressive import flare_autoregressive_stablemax_triton
    _case("stablemax decoder", mode)
    B, N, H, M, D = 2, 150, 2, 32, 16
    q, k, v = seeded(71, B, N, H, M, D, D, torch.float32, q_std=D ** -0.5)
    g = torch.Generator().manual_seed(72)
    qd = torch.randn(k.shape, generator=g) if mode in ("sep_q", "both") else None
    kd = torch.randn(q.shape, generator=g) * D ** -0.5 if mode in ("sep_k", "both") else None
    y = flare_autoregressive_stablemax_triton(q.to(DEV), k.to(DEV), v.to(DEV), power=2.0, scale=0.4,
                                              Q_dec=None if qd is None else qd.to(DEV),
                                              K_dec=None if kd is None else kd.to(DEV))
    ref = O.brute_stablemax(q, k, v, power=2.0, scale=0.4, Q_dec=qd, K_dec=kd)
    assert_parity(y, ref, torch.float32, f"stablemax decoder {mode}")


def test_stablemax_reference_sizes_bf16():
    """A 128 x 64 latent bank over 1024 tokens (the reference's default Triton chunk of 128)."""
    from causal_flare.autoregressive import flare_autoregressive_stablemax_triton
    _case("stablemax 128x64")
    B, N, H, M, D = 1, 1024, 4, 128, 64
    q, k, v = seeded(73, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    y = flare_autoregressive_stablemax_triton(q.to(DEV), k.to(DEV), v.to(DEV))
    ref = O.brute_stablemax(q, k, v, power=2.0)
    assert_parity(y, ref, torch.bfloat16, "stablemax 128x64")
    assert np.isfinite(y.float().cpu().numpy()).all()
