"""Token-recurrent causal FLARE entry point on MI355X.

Drop-in for the reference's experimental ``flare_recurrent_triton`` /
``RecurrentFLARE`` (``causal_flare/autoregressive/recurrent.py:288-416,
1191-1204``).  The recurrent form computes the same output as the chunked
forward -- per token, the online-softmax update of (m, d, U) for every latent
and the softmax readout over the latents (``flare_recurrent_pytorch``,
recurrent.py:17-57) -- so it runs on the same HIP kernels: the chunked forward
(``flare_ar_forward``) and its backward (``flare_ar_backward``).  Kept as in
the reference: the argument list, validation and its messages, the output
layout ``[B, H, T, D]`` in ``Q.dtype``, and differentiability.  The
``block_m`` / ``block_d`` / ``block_t`` tile arguments (and their
FLARE_RECURRENT_BLOCK_* environment overrides) are validated as the reference
validates them (recurrent.py:60-116); they do not change the result.
"""
from __future__ import annotations

import os

import torch
import torch.autograd as autograd

from .._common import _require_gpu, _resolve_attn_scale
from .._reference_utils import resolve_flare_causal_decode_inputs
from .training import _decoder_args, _resolve_chunk_size, run_chunked_backward, run_chunked_forward


def _env_int(name):
    v = os.environ.get(name, "").strip()
    return int(v) if v else None


def _check_block_d_k(D, block_d):
    """recurrent.py:60-83."""
    bd = int(block_d) if block_d is not None else _env_int("FLARE_RECURRENT_BLOCK_D")
    bd = min(bd if bd is not None else (D if D <= 128 else 64), D)
    if bd % 16 != 0:
        raise ValueError(f"Recurrent BLOCK_D must be a multiple of 16. Got BLOCK_D={bd}")
    bk = _env_int("FLARE_RECURRENT_BLOCK_K")
    bk = min(bk if bk is not None else (D if bd == D else 64), D)
    if bk % 16 != 0:
        raise ValueError(f"Recurrent BLOCK_K must be a multiple of 16. Got BLOCK_K={bk}")


def _check_block_t(block_t):
    """recurrent.py:86-101."""
    bt = int(block_t) if block_t is not None else _env_int("FLARE_RECURRENT_BLOCK_T")
    bt = 16 if bt is None else bt
    if bt == 1:
        return
    if bt % 16 != 0:
        raise ValueError(f"Recurrent BLOCK_T must be 1 or a multiple of 16. Got BLOCK_T={bt}")
    if bt not in (16, 32):
        raise ValueError(f"Recurrent BLOCK_T currently supports [1, 16, 32]. Got BLOCK_T={bt}")


def _check_block_m(M, block_m):
    """recurrent.py:104-116."""
    bm = int(block_m) if block_m is not None else _env_int("FLARE_RECURRENT_BLOCK_M")
    bm = min(bm if bm is not None else M, M)
    if bm % 16 != 0:
        raise ValueError(f"Recurrent BLOCK_M must be a multiple of 16. Got BLOCK_M={bm}")


class RecurrentFLARE(autograd.Function):
    """reference recurrent.py:288-416; Y [B, H, T, D] in Q.dtype."""

    @staticmethod
    def forward(ctx, Q, K, V, scale=None, block_m=None, block_d=None, Q_dec=None, K_dec=None, block_t=None):
        if Q.dim() != 3 or K.dim() != 4 or V.dim() != 4:
            raise ValueError(
                "Recurrent FLARE expects Q [H, M, D] and K/V [B, N, H, D]. "
                f"Got Q.dim()={Q.dim()}, K.dim()={K.dim()}, V.dim()={V.dim()}"
            )
        if K.size() != V.size():
            raise ValueError(f"K and V must have the same shape. Got K.shape={K.shape} and V.shape={V.shape}")
        if Q.size(0) != K.size(2) or Q.size(2) != K.size(3):
            raise ValueError(
                "Expected Q [H, M, D] and K/V [B, N, H, D] with matching H,D. "
                f"Got Q.shape={Q.shape} and K.shape={K.shape}"
            )
        H, M, D = Q.size()
        B, T, _, _ = K.size()
        scale = _resolve_attn_scale(scale, D)
        Q_dec_r, K_dec_r, sep_q, sep_k, shared = resolve_flare_causal_decode_inputs(Q, K, Q_dec, K_dec)
        if (M % 16) != 0 or (D % 16) != 0:
            raise ValueError(f"RecurrentFLARE requires M and D be multiples of 16. Got M={M}, D={D}")
        _check_block_m(M, block_m)
        _check_block_d_k(D, block_d)
        _check_block_t(block_t)
        _require_gpu("flare_recurrent_triton", Q, K, V, Q_dec, K_dec)
        qd = kd = None
        if T == 0:
            Y = torch.empty((B, 0, H, D), device=K.device, dtype=Q.dtype)
        else:
            _, chunk = _resolve_chunk_size(None, B, T, H, M, D)
            qd, kd = (None, None) if shared else _decoder_args(Q, K, Q_dec_r, K_dec_r, sep_q, sep_k)
            Y, _ = run_chunked_forward(Q, K, V, qd, kd, scale=scale, chunk=chunk, out_dtype=Q.dtype)
        ctx.scale = scale
        ctx.save_for_backward(Q, K, V, qd, kd, Y)
        return Y.permute(0, 2, 1, 3).contiguous()

    @staticmethod
    def backward(ctx, dY):
        Q, K, V, qd, kd, Y = ctx.saved_tensors
        g = None if dY is None else dY.permute(0, 2, 1, 3)
        dq, dk, dv, dqd, dkd = run_chunked_backward(Q, K, V, qd, kd, Y, g, scale=ctx.scale)
        return dq, dk, dv, None, None, None, dqd, dkd, None


def flare_recurrent_triton(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    scale: float | None = None,
    *,
    block_m: int | None = None,
    block_d: int | None = None,
    Q_dec: torch.Tensor | None = None,
    K_dec: torch.Tensor | None = None,
    block_t: int | None = None,
):
    """Recurrent FLARE: Q [H,M,D], K/V [B,T,H,D] -> Y [B,H,T,D] (reference recurrent.py:1191-1204)."""
    return RecurrentFLARE.apply(Q, K, V, scale, block_m, block_d, Q_dec, K_dec, block_t)
