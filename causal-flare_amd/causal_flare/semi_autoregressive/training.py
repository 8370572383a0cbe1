"""Block-causal (semi-autoregressive) causal FLARE forward on MI355X.

Drop-in for ``flare_semi_autoregressive_trition`` / ``SemiAutoRegressiveFLARE``
(``causal_flare/semi_autoregressive/training.py:3990-4106``): token t of block
g attends to every token of blocks <= g.  Returns ``(Y, {"LSE_dec": [B,H,N],
"LSE_enc": [B,H,NB,M]})`` and, with ``profile=True``, a third timings dict.
Validation (``semi_autoregressive/reference.py:17-51``) runs before the device
check, so its errors are raised for CPU tensors too.  The backward
(reference ``_semi_autoregressive_backward_impl``, training.py:3768-3988) runs
as HIP kernels through ``flare_semi_ar_backward``.
"""
from __future__ import annotations

import math

import torch
import torch.autograd as autograd

from .. import _lib
from .._common import (
    _PhaseTimer,
    _compute_dtype,
    _normalize_input_precision,
    _refresh_profile_totals,
    _resolve_attn_scale,
)
from .._reference_utils import resolve_flare_causal_decode_inputs, validate_flare_qkv_layouts

_SUPPORTED_BLOCK_CAUSAL_CHUNK_SIZES = (16, 32, 64, 128)


def _validate_block_causal_config(*, N: int, block_size, chunk_size, name: str):
    """Block/chunk rules and messages of semi_autoregressive/reference.py:17-51."""
    if block_size is None:
        raise ValueError(f"{name} requires block_size to be specified explicitly.")
    if chunk_size is None:
        raise ValueError(f"{name} requires chunk_size to be specified explicitly.")
    block_size = int(block_size)
    chunk_size = int(chunk_size)
    if block_size <= 0:
        raise ValueError(f"{name} requires block_size > 0. Got block_size={block_size}.")
    if block_size % 16 != 0:
        raise ValueError(f"{name} requires block_size to be a positive multiple of 16. Got block_size={block_size}.")
    if chunk_size not in _SUPPORTED_BLOCK_CAUSAL_CHUNK_SIZES:
        raise ValueError(
            f"{name} currently supports chunk_size in {_SUPPORTED_BLOCK_CAUSAL_CHUNK_SIZES}. Got chunk_size={chunk_size}."
        )
    if N % block_size != 0:
        raise ValueError(
            f"{name} requires sequence length N to be an exact multiple of block_size. Got N={N}, block_size={block_size}."
        )
    if block_size % chunk_size != 0:
        raise ValueError(
            f"{name} requires block_size to be an integer multiple of chunk_size so blocks align with chunk summaries. "
            f"Got block_size={block_size}, chunk_size={chunk_size}."
        )
    num_blocks = math.ceil(N / block_size) if N > 0 else 0
    num_chunks = math.ceil(N / chunk_size) if N > 0 else 0
    return block_size, chunk_size, num_blocks, num_chunks, block_size // chunk_size


def _semi_autoregressive_forward(Q, K, V, *, block_size, chunk_size, scale=None, input_precision=None,
                                 profile=False, Q_dec=None, K_dec=None, saved=None):
    """Forward launch; when ``saved`` is a dict it receives what the backward needs."""
    name = "SemiAutoRegressiveFLARE"
    B, N, H, M, D_score, D_value = validate_flare_qkv_layouts(Q, K, V, name=name)
    block_size, chunk_size, NB, _, _ = _validate_block_causal_config(
        N=N, block_size=block_size, chunk_size=chunk_size, name=name)
    if Q.device.type != "cuda" or K.device.type != "cuda" or V.device.type != "cuda":
        raise ValueError("SemiAutoRegressiveFLARE Triton forward requires CUDA tensors.")
    Q_dec, K_dec, sep_q, sep_k, shared = resolve_flare_causal_decode_inputs(Q, K, Q_dec, K_dec)
    scale = _resolve_attn_scale(scale, D_score)
    _normalize_input_precision(input_precision)
    device = K.device
    qd = None if (shared or not sep_q or Q_dec is K) else Q_dec
    kd = None if (shared or not sep_k or K_dec is Q) else K_dec
    cdt = _compute_dtype(Q, K, V, qd, kd)
    q, k, v = (t.to(cdt).contiguous() for t in (Q, K, V))
    qd = None if qd is None else qd.to(cdt).contiguous()
    kd = None if kd is None else kd.to(cdt).contiguous()
    Y = torch.empty((B, N, H, D_value), device=device, dtype=V.dtype)
    lse_dec = torch.empty((B, H, N), device=device, dtype=torch.float32)
    lse_enc = torch.empty((B, H, NB, M), device=device, dtype=torch.float32)
    lib = _lib.lib()
    size_fn = (lib.flare_semi_ar_workspace_size if qd is None and kd is None
               else lib.flare_semi_ar_workspace_size_sep)
    nbytes = size_fn(B, N, H, M, D_value, block_size)
    ws = torch.empty(max(nbytes, 1), device=device, dtype=torch.uint8)
    P = _lib.ptr
    launch = lambda: lib.flare_semi_ar_forward(
        P(q), P(k), P(v), P(qd), P(kd), _lib.dtype_code(cdt), B, N, H, M, D_score, D_value,
        float(scale), block_size, P(Y), _lib.dtype_code(V.dtype), P(lse_dec), P(lse_enc), P(ws),
        nbytes, _lib.stream_of(device))
    profile_data = {"forward": {}, "backward": {}} if profile else None
    rc = _PhaseTimer(device, profile_data["forward"] if profile else None)("semi_ar_forward", launch)
    _lib.check(rc, "flare_semi_ar_forward")
    aux = {"LSE_dec": lse_dec, "LSE_enc": lse_enc}
    if saved is not None:
        saved.update(qd=qd, kd=kd, Y=Y, scale=scale, block=block_size)
    if profile:
        _refresh_profile_totals(profile_data)
        return Y, aux, profile_data
    return Y, aux


def run_semi_backward(Q, K, V, qd, kd, Y, dY, *, scale, block):
    """Launch flare_semi_ar_backward; returns (dQ, dK, dV, dQ_dec, dK_dec) in the
    inputs' dtypes (None for a decoder tensor that was not separate)."""
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    if dY is None:
        return None, None, None, None, None
    if N == 0:
        return tuple(None if t is None else torch.zeros_like(t) for t in (Q, K, V, qd, kd))
    if M > 256 or Dk > 256 or Dv > 512:
        raise NotImplementedError(
            f"The MI355X semi-autoregressive FLARE backward supports M <= 256, D_score <= 256 and D_value <= 512; "
            f"got M={M}, D_score={Dk}, D_value={Dv}."
        )
    device = K.device
    cdt = _compute_dtype(Q, K, V, qd, kd)
    prep = lambda t: None if t is None else t.to(cdt).contiguous()
    q, k, v, qdc, kdc, y, dy = (prep(t) for t in (Q, K, V, qd, kd, Y, dY))
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dqd = torch.empty_like(qdc) if qdc is not None else None
    dkd = torch.empty_like(kdc) if kdc is not None else None
    lib = _lib.lib()
    nbytes = lib.flare_semi_ar_backward_workspace_size(B, N, H, M, Dk, Dv, block)
    ws = torch.empty(nbytes, device=device, dtype=torch.uint8)
    P = _lib.ptr
    rc = lib.flare_semi_ar_backward(P(q), P(k), P(v), P(qdc), P(kdc), _lib.dtype_code(cdt), B, N, H, M, Dk, Dv,
                                    float(scale), block, P(y), P(dy), P(dq), P(dk), P(dv), P(dqd), P(dkd), P(ws),
                                    nbytes, _lib.stream_of(device))
    _lib.check(rc, "flare_semi_ar_backward")
    cast = lambda g, ref: None if g is None else g.to(ref.dtype)
    return cast(dq, Q), cast(dk, K), cast(dv, V), cast(dqd, qd), cast(dkd, kd)


class SemiAutoRegressiveFLARE(autograd.Function):
    """Forward of block-causal FLARE (reference semi training.py:3990-4079)."""

    @staticmethod
    def forward(ctx, Q, K, V, scale=None, block_size=None, chunk_size=None, input_precision=None,
                profile=False, Q_dec=None, K_dec=None):
        saved = {}
        out = _semi_autoregressive_forward(Q, K, V, block_size=block_size, chunk_size=chunk_size, scale=scale,
                                           input_precision=input_precision, profile=profile, Q_dec=Q_dec,
                                           K_dec=K_dec, saved=saved)
        ctx.scale = saved.get("scale")
        ctx.block = saved.get("block")
        ctx.save_for_backward(Q, K, V, saved.get("qd"), saved.get("kd"), saved.get("Y"))
        return out

    @staticmethod
    def backward(ctx, dY, *unused):
        """Gradients of Q, K, V (and Q_dec, K_dec when separate): reference
        _semi_autoregressive_backward_impl (semi training.py:3768-3988)."""
        Q, K, V, qd, kd, Y = ctx.saved_tensors
        dq, dk, dv, dqd, dkd = run_semi_backward(Q, K, V, qd, kd, Y, dY, scale=ctx.scale, block=ctx.block)
        return dq, dk, dv, None, None, None, None, None, dqd, dkd


def flare_semi_autoregressive_trition(Q, K, V, *, block_size, chunk_size, scale=None, input_precision=None,
                                      profile: bool = False, Q_dec=None, K_dec=None):
    """Block-causal FLARE forward (reference semi training.py:4082-4106)."""
    return SemiAutoRegressiveFLARE.apply(Q, K, V, scale, block_size, chunk_size, input_precision, profile,
                                         Q_dec, K_dec)
