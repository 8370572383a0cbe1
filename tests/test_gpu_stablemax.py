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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("power", [1.0, 2.0, 4.0, 2.5])
@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
def test_stablemax_mfma_forward(dtype, power, M, D):
    """The MFMA path (bf16 / fp16, M in {128, 256}, D in {64, 128}): decoder softmax pass,
    then chunk_output_tr with the stablemax transform; ragged N, the library's chunk and an
    explicit one, shared and separate decoder tensors."""
    from causal_flare.autoregressive import flare_autoregressive_stablemax_triton
    _case("stablemax mfma", dtype, power, M, D)
    B, N, H = 2, 1000, 2
    q, k, v = seeded(74 + M, B, N, H, M, D, D, dtype, q_std=D ** -0.5)
    # (the chunked fp64 form, pinned to brute_stablemax in tests/test_oracle.py: the
    # per-token definition is quadratic in N)
    ref = O.stablemax_chunked(q, k, v, power=power)
    for chunk in (None, 256):
        y = flare_autoregressive_stablemax_triton(q.to(DEV), k.to(DEV), v.to(DEV), power=power, chunk_size=chunk)
        assert_parity(y, ref, dtype, f"stablemax mfma power={power} {M}x{D} chunk={chunk}")
    g = torch.Generator().manual_seed(75)
    qd = torch.randn(k.shape, generator=g).to(dtype)
    kd = (torch.randn(q.shape, generator=g) * D ** -0.5).to(dtype)
    y = flare_autoregressive_stablemax_triton(q.to(DEV), k.to(DEV), v.to(DEV), power=power, Q_dec=qd.to(DEV),
                                              K_dec=kd.to(DEV))
    ref = O.stablemax_chunked(q, k, v, power=power, Q_dec=qd, K_dec=kd)
    assert_parity(y, ref, dtype, f"stablemax mfma separate decoder power={power} {M}x{D}")


# --------------------------------------------------------------------------
# Backward (C flare_stablemax_backward) against fp64 autograd of the definition
# (O.stablemax_grads, pinned by finite differences in tests/test_oracle.py).
# Bar: the reference's own (test_stablemax.py:428-482, fp32 inputs: rtol = atol
# = 2e-3, 3e-3 for powers 3 and 4); 16-bit inputs: max |g - g_ref| <= 2e-2 of
# max |g_ref| per tensor, as the token-causal backward tests.
# --------------------------------------------------------------------------
def _stablemax_grads_gpu(q, k, v, qd, kd, dy, power, scale, chunk):
    from causal_flare.autoregressive import flare_autoregressive_stablemax_triton
    leaves = [None if t is None else t.to(DEV).requires_grad_(True) for t in (q, k, v, qd, kd)]
    y = flare_autoregressive_stablemax_triton(leaves[0], leaves[1], leaves[2], scale=scale, chunk_size=chunk,
                                              Q_dec=leaves[3], K_dec=leaves[4], power=power)
    (y.float() * dy.to(DEV)).sum().backward()
    return [None if t is None else t.grad for t in leaves]


def _grad_check(got, ref, names, dtype, tol, what):
    for g, r, n in zip(got, ref, names):
        if r is None:
            continue
        a = g.float().cpu().numpy()
        assert np.isfinite(a).all(), f"{what} {n}: non-finite gradient"
        if dtype == torch.float32:
            np.testing.assert_allclose(a, r, rtol=tol, atol=tol, err_msg=f"{what} {n}")
        else:
            err = float(np.abs(a - r).max() / max(np.abs(r).max(), 1e-2))
            assert err <= 2e-2, f"{what} {n}: max|g - ref| / max|ref| = {err:.3e}"


@pytest.mark.parametrize("power", [2.0, 3.0, 4.0])
def test_stablemax_backward_reference_case(power):
    """The reference's backward test shape (test_stablemax.py:428-482): B=2, H=2, M=32,
    N=128, D=32, chunk 64, separate decoder tensors, fp32."""
    _case("stablemax backward", power)
    g = torch.Generator().manual_seed(4)
    B, H, M, N, D = 2, 2, 32, 128, 32
    q, k, v = (torch.randn(s, generator=g) for s in ((H, M, D), (B, N, H, D), (B, N, H, D)))
    qd, kd = torch.randn((B, N, H, D), generator=g), torch.randn((H, M, D), generator=g)
    dy = torch.randn((B, N, H, D), generator=g)
    got = _stablemax_grads_gpu(q, k, v, qd, kd, dy, power, D ** -0.5, 64)
    ref = O.stablemax_grads(q, k, v, dy, power, D ** -0.5, qd, kd)
    _grad_check(got, ref, ("dQ", "dK", "dV", "dQ_dec", "dK_dec"), torch.float32,
                2e-3 if power == 2.0 else 3e-3, f"stablemax backward power={power}")


@pytest.mark.parametrize("mode", ["shared", "sep_q", "sep_k"])
@pytest.mark.parametrize("power", [1.0, 2.5])
def test_stablemax_backward_decoder_modes(mode, power):
    """Shared decoder weights (the decoder share folds into dQ / dK), one separate decoder
    tensor, a non-integer power, ragged N (not a multiple of the 16-token chunk)."""
    _case("stablemax backward modes", mode, power)
    B, N, H, M, D, Dv = 2, 77, 2, 48, 16, 32
    g = torch.Generator().manual_seed(81)
    q = torch.randn((H, M, D), generator=g) * D ** -0.5 * 2
    k, v = torch.randn((B, N, H, D), generator=g), torch.randn((B, N, H, Dv), generator=g)
    qd = torch.randn((B, N, H, D), generator=g) if mode == "sep_q" else None
    kd = torch.randn((H, M, D), generator=g) * 0.3 if mode == "sep_k" else None
    dy = torch.randn((B, N, H, Dv), generator=g)
    got = _stablemax_grads_gpu(q, k, v, qd, kd, dy, power, 0.5, None)
    ref = O.stablemax_grads(q, k, v, dy, power, 0.5, qd, kd)
    _grad_check(got, ref, ("dQ", "dK", "dV", "dQ_dec", "dK_dec"), torch.float32, 2e-3,
                f"stablemax backward {mode} power={power}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_stablemax_backward_16bit_large_bank(dtype):
    """A 256 x 128 bank (the 8-token chunk, past the 60 KiB row budget of 16) and a
    128 x 64 bank, 16-bit inputs."""
    for (B, N, H, M, D) in ((1, 96, 2, 256, 128), (2, 200, 2, 128, 64)):
        _case("stablemax backward 16-bit", dtype, M, D)
        q, k, v = seeded(90 + M, B, N, H, M, D, D, dtype, q_std=D ** -0.5)
        g = torch.Generator().manual_seed(91)
        dy = torch.randn((B, N, H, D), generator=g)
        got = _stablemax_grads_gpu(q, k, v, None, None, dy, 2.0, None, None)
        ref = O.stablemax_grads(q, k, v, dy, 2.0, None, None, None)
        _grad_check(got, ref, ("dQ", "dK", "dV"), dtype, None, f"stablemax backward {dtype} {M}x{D}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_stablemax_backward_other_shapes(dtype):
    """M and D_score not multiples of 16: the chunked fp32 replay kernels (every
    other shape runs the softmax backward's pipeline with log2 s(a) as scores)."""
    B, N, H, M, D, Dv = 2, 70, 2, 40, 24, 32
    _case("stablemax backward other shapes", dtype, M, D, Dv)
    g = torch.Generator().manual_seed(93)
    q = (torch.randn((H, M, D), generator=g) * D ** -0.5).to(dtype)
    k, v = torch.randn((B, N, H, D), generator=g).to(dtype), torch.randn((B, N, H, Dv), generator=g).to(dtype)
    dy = torch.randn((B, N, H, Dv), generator=g)
    got = _stablemax_grads_gpu(q, k, v, None, None, dy, 3.0, None, None)
    ref = O.stablemax_grads(q, k, v, dy, 3.0, None, None, None)
    _grad_check(got, ref, ("dQ", "dK", "dV"), dtype, 3e-3, f"stablemax backward {dtype} {M}x{D}x{Dv}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_stablemax_backward_long_wide_scores(dtype, monkeypatch):
    """Many 32-token backward chunks and wide scores (|a| up to about 10, power 4:
    weights spanning about 2^28), shared decoder; the chunk starting states walked over
    256-token chunks (four tiles each)."""
    B, N, H, M, D = 1, 700, 2, 128, 64
    _case("stablemax backward long", dtype)
    monkeypatch.setenv("FLARE_BWD_WALK_CHUNK", "256")
    q, k, v = seeded(95, B, N, H, M, D, D, dtype, q_std=2.5)   # a = scale k.q ~ N(0, 2.5^2)
    g = torch.Generator().manual_seed(96)
    dy = torch.randn((B, N, H, D), generator=g)
    got = _stablemax_grads_gpu(q, k, v, None, None, dy, 4.0, None, None)
    ref = O.stablemax_grads(q, k, v, dy, 4.0, None, None, None)
    _grad_check(got, ref, ("dQ", "dK", "dV"), dtype, 3e-3, f"stablemax backward long {dtype}")
