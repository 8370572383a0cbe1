"""Semi-autoregressive (block-causal) cached prefill and block decode on MI355X.

The reference ships these entry points as stubs that raise
``NotImplementedError`` (``causal_flare/semi_autoregressive/inference.py:5-36``).
Here they are implemented with the same names and keyword arguments, plus a
``block_size`` keyword:

* The tokens of a prefill form whole blocks of ``block_size`` tokens.  As in
  ``flare_semi_autoregressive_trition`` (semi ``training.py:4082-4088``),
  ``block_size`` is required: a prefill without it raises ``ValueError`` (a
  default of one block per call would let every prompt token read later tokens).
  Every token of a block reads the latent state after its whole block, as in the
  block-causal forward (``semi_autoregressive/reference.py:560-597``).  A block
  decode step is one block: the ``T`` tokens of the call.
* The state is the autoregressive cache ``{"m": [B,H,M], "d": [B,H,M],
  "u": [B,H,M,Dv]}`` (fp32; ``autoregressive/inference.py:66-120``): it stands for
  every earlier block, so a semi-AR prefill can continue an autoregressive one and
  the other way round.
* Prefill returns ``(Y, new_state)``; decode runs one block (``K, V`` as
  ``[B, T, H, D]``, or ``[B, H, D]`` for one token) and updates the caller's state
  tensors in place, returning ``(Y, state)`` with the same tensors, as the
  autoregressive decode does.
* ``scale=None`` resolves to ``D**-0.5``, as in ``flare_semi_autoregressive_trition``.

A block must hold a multiple of 16 tokens (the block-causal kernels' rule); a
one-token decode step is the autoregressive step.  The backward is not
implemented (the classes raise, as the reference's do).
"""
from __future__ import annotations

import torch
import torch.autograd as autograd

from .. import _lib
from .._common import _compute_dtype, _resolve_attn_scale
from .._reference_utils import resolve_flare_causal_decode_inputs, validate_flare_qkv_layouts
from ..autoregressive.inference import _canonicalize_flare_state, flare_autoregressive_decode_triton


def _semi_cached(Q, K, V, *, state, scale, Q_dec, K_dec, block_size, name):
    """One launch of flare_semi_ar_forward_state; returns (Y, canonical input state, state after)."""
    B, N, H, M, D_score, D_value = validate_flare_qkv_layouts(Q, K, V, name=name)
    if block_size is None:
        raise ValueError(f"{name} requires block_size (tokens per block).")
    block = int(block_size)
    if block <= 0 or block % 16 != 0:
        raise ValueError(f"{name} requires block_size to be a positive multiple of 16. Got block_size={block}.")
    if N % block != 0:
        raise ValueError(
            f"{name} requires the number of tokens to be an exact multiple of block_size. Got N={N}, "
            f"block_size={block}."
        )
    if Q.device.type != "cuda" or K.device.type != "cuda" or V.device.type != "cuda":
        raise RuntimeError(f"{name} requires CUDA tensors.")
    Q_dec, K_dec, sep_q, sep_k, shared = resolve_flare_causal_decode_inputs(Q, K, Q_dec, K_dec)
    scale = _resolve_attn_scale(scale, D_score)
    device = K.device
    st = _canonicalize_flare_state(state, B, H, M, D_value, device) if state is not None else None
    qd = None if (shared or not sep_q or Q_dec is K) else Q_dec
    kd = None if (shared or not sep_k or K_dec is Q) else K_dec
    cdt = _compute_dtype(Q, K, V, qd, kd)
    q, k, v = (t.to(cdt).contiguous() for t in (Q, K, V))
    qd = None if qd is None else qd.to(cdt).contiguous()
    kd = None if kd is None else kd.to(cdt).contiguous()
    Y = torch.empty((B, N, H, D_value), device=device, dtype=V.dtype)
    out = {
        "m": torch.empty((B, H, M), device=device, dtype=torch.float32),
        "d": torch.empty((B, H, M), device=device, dtype=torch.float32),
        "u": torch.empty((B, H, M, D_value), device=device, dtype=torch.float32),
    }
    src = None if st is None else {key: st[key].contiguous() for key in ("m", "d", "u")}
    lib = _lib.lib()
    size_fn = (lib.flare_semi_ar_workspace_size if qd is None and kd is None
               else lib.flare_semi_ar_workspace_size_sep)
    nbytes = size_fn(B, N, H, M, D_value, block)
    ws = torch.empty(max(nbytes, 1), device=device, dtype=torch.uint8)
    P = _lib.ptr
    rc = lib.flare_semi_ar_forward_state(
        P(q), P(k), P(v), P(qd), P(kd), _lib.dtype_code(cdt), B, N, H, M, D_score, D_value, float(scale), block,
        P(src["m"]) if src else None, P(src["d"]) if src else None, P(src["u"]) if src else None,
        P(out["m"]), P(out["d"]), P(out["u"]), P(Y), _lib.dtype_code(V.dtype), P(ws), nbytes,
        _lib.stream_of(device))
    _lib.check(rc, "flare_semi_ar_forward_state")
    return Y, st, out


def flare_semi_autoregressive_prefill_trition(Q, K, V, *, state=None, scale=None, attention_mask=None, Q_dec=None,
                                              K_dec=None, block_size=None):
    """Block-causal prefill of ``K, V [B, T, H, D]`` continuing ``state``; returns ``(Y, state)``.

    ``attention_mask`` is accepted for the stub's signature; a mask that drops
    tokens is not supported here (NotImplementedError), an all-ones mask is ignored.
    """
    name = "flare_semi_autoregressive_prefill_trition"
    if attention_mask is not None and not bool((attention_mask != 0).all()):
        raise NotImplementedError(f"{name}: attention_mask that drops tokens is not supported.")
    Y, _, new_state = _semi_cached(Q, K, V, state=state, scale=scale, Q_dec=Q_dec, K_dec=K_dec,
                                   block_size=block_size, name=name)
    return Y, new_state


def flare_semi_autoregressive_decode_trition(Q, K, V, *, state=None, scale=None, Q_dec=None, K_dec=None):
    """One block step: ``K, V [B, T, H, D]`` (T a multiple of 16) or one token ``[B, H, D]``
    / ``[B, 1, H, D]``; the caller's fp32 state tensors are updated in place."""
    name = "flare_semi_autoregressive_decode_trition"
    single = K.dim() == 3 or (K.dim() == 4 and K.shape[1] == 1)
    if single:
        # a one-token block reads the state after its own token: the autoregressive step
        D = K.shape[-1]
        return flare_autoregressive_decode_triton(Q, K, V, state=state, scale=_resolve_attn_scale(scale, D),
                                                  Q_dec=Q_dec, K_dec=K_dec)
    Y, st, out = _semi_cached(Q, K, V, state=state, scale=scale, Q_dec=Q_dec, K_dec=K_dec, block_size=K.shape[1],
                              name=name)
    if st is None:
        return Y, out
    for key in ("m", "d", "u"):
        st[key].copy_(out[key])
    return Y, st


class SemiAutoRegressivePrefillFLARE(autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, state=None, scale=None, attention_mask=None, Q_dec=None, K_dec=None, block_size=None):
        return flare_semi_autoregressive_prefill_trition(Q, K, V, state=state, scale=scale,
                                                         attention_mask=attention_mask, Q_dec=Q_dec, K_dec=K_dec,
                                                         block_size=block_size)

    @staticmethod
    def backward(ctx, dY, dState=None):
        raise NotImplementedError("SemiAutoRegressivePrefillFLARE backward is not implemented yet.")


class SemiAutoRegressiveDecodeFLARE(autograd.Function):
    @staticmethod
    def forward(ctx, Q, K, V, state=None, scale=None, Q_dec=None, K_dec=None):
        return flare_semi_autoregressive_decode_trition(Q, K, V, state=state, scale=scale, Q_dec=Q_dec, K_dec=K_dec)

    @staticmethod
    def backward(ctx, dY, dState=None):
        raise NotImplementedError("SemiAutoRegressiveDecodeFLARE backward is not implemented yet.")
