"""Stablemax causal FLARE on MI355X: the non-write-gated path of the reference's
``flare_autoregressive_stablemax_triton`` (``causal_flare/autoregressive/
stablemax_triton.py:1707-2055, 2423-2468``).

The encoder weights are the stablemax transform of the scores instead of their
exponential, the decoder weights stay a softmax over the latents:

    y_t = sum_m softmax_m(scale qd_t . kd_m) *
          (sum_{tau<=t} s(a_tau,m) v_tau) / (sum_{tau<=t} s(a_tau,m)),
    a_tau,m = scale k_tau . q_m,   s(x) = (1+x)^p (x >= 0), (1-x)^-p (x < 0).

It runs in C ``flare_stablemax_forward``: chunk sums of s(a) and s(a) v, their
exclusive scan, and the replay with the latent-softmax readout.  bf16 / fp16
inputs with M in {128, 256} and D_score = D_value in {64, 128} take the MFMA
kernels (the decoder softmax pass, then the producer / consumer output kernel
with the stablemax transform of the scores, log2 s(a) against lazy per-latent
references, fp32 accumulation); other dtypes and shapes, and explicit chunk
sizes that are not a multiple of 32, the fp32 chunk kernels.  With no
``chunk_size`` the library picks the chunk (one round of workgroups); the
output has V's dtype.  Kept as in the reference: the argument list, the
``NotImplementedError`` for the options its Triton path does not implement
(``eps``, ``profile``, recurrent ``state``, ``attention_mask``,
``return_state``, write gates) and the chunk-size rule (a multiple of 16).
The backward (``stablemax_triton.py:1981-2420``, C ``flare_stablemax_backward``)
is the softmax backward's pipeline with the encoder weight s(a) in place of e^a
(scores as log2 s(a), score gradients times p / (1 + |a|)) when M, D_score and
D_value are multiples of 16, and a chunked fp32 replay otherwise.  It supports
M <= 256 and head dims up to 256 (``NotImplementedError`` beyond).
"""
from __future__ import annotations

import os

import torch
import torch.autograd as autograd

from .. import _lib
from .._common import _normalize_input_precision, _require_gpu, _resolve_attn_scale
from .._reference_utils import resolve_flare_causal_decode_inputs, validate_flare_qkv_layouts


def _resolve_stablemax_chunk_size(N, M, D_score, D_value, chunk_size):
    """stablemax.py:27-42 (the Triton path's default chunk)."""
    if chunk_size is None:
        env_chunk = os.environ.get("FLARE_PYTORCH_CHUNK_SIZE", "")
        chunk_size = int(env_chunk) if env_chunk else None
    if chunk_size is not None:
        return int(chunk_size)
    if D_value > 128 and (M >= 256 or D_score >= 128):
        return 64
    if D_score <= 32 and M <= 64:
        return 64
    return 128


def _stablemax_forward(Q, K, V, Q_dec, K_dec, scale, chunk_size, power, input_precision, ctx=None):
    B, N, H, M, D_score, D_value = validate_flare_qkv_layouts(Q, K, V, name="Stablemax Triton FLARE")
    scale_f = _resolve_attn_scale(scale, D_score)
    power_f = float(power)
    _normalize_input_precision(input_precision)
    _, _, sep_q, sep_k, shared = resolve_flare_causal_decode_inputs(Q, K, Q_dec, K_dec)
    chunk = _resolve_stablemax_chunk_size(N, M, D_score, D_value, chunk_size)
    # (the reference's default chunk is a Triton tile size; without an explicit one the
    # library chooses, which changes rounding only)
    lib_chunk = chunk if (chunk_size is not None or os.environ.get("FLARE_PYTORCH_CHUNK_SIZE")) else 0
    if chunk % 16 != 0:
        raise ValueError(
            "FLAREAutoregressiveStablemaxTriton requires a chunk size divisible by 16. "
            f"Got chunk_size={chunk}."
        )
    if not (power_f > 0.0) or power_f != power_f or power_f == float("inf"):
        raise ValueError(f"Stablemax power must be positive and finite. Got power={power}.")
    out_dtype = V.dtype
    if N == 0:
        return torch.empty((B, 0, H, D_value), device=V.device, dtype=out_dtype)
    _require_gpu("flare_autoregressive_stablemax_triton", Q, K, V, Q_dec, K_dec)
    qd = Q_dec if (not shared and sep_q and Q_dec is not K) else None
    kd = K_dec if (not shared and sep_k and K_dec is not Q) else None
    dts = [t.dtype for t in (Q, K, V, qd, kd) if t is not None]
    cdt = dts[0] if all(d == dts[0] for d in dts) and dts[0] in (torch.bfloat16, torch.float16) else torch.float32
    q, k, v = (t.to(cdt).contiguous() for t in (Q, K, V))
    qd = None if qd is None else qd.to(cdt).contiguous()
    kd = None if kd is None else kd.to(cdt).contiguous()
    Y = torch.empty((B, N, H, D_value), device=V.device, dtype=out_dtype)
    lib = _lib.lib()
    nbytes = lib.flare_ar_forward_workspace_size_sep(B, N, H, M, D_value, lib_chunk)
    ws = torch.empty(max(nbytes, 1), device=V.device, dtype=torch.uint8)
    P = _lib.ptr
    rc = lib.flare_stablemax_forward(P(q), P(k), P(v), P(qd), P(kd), _lib.dtype_code(cdt), B, N, H, M, D_score,
                                     D_value, float(scale_f), lib_chunk, power_f, P(Y), _lib.dtype_code(out_dtype),
                                     P(ws), nbytes, _lib.stream_of(V.device))
    _lib.check(rc, "flare_stablemax_forward")
    if ctx is not None:
        ctx.save_for_backward(q, k, v, qd, kd, Y)
        ctx.meta = (Q.dtype, K.dtype, V.dtype, Q_dec.dtype, K_dec.dtype, cdt, float(scale_f), power_f)
    return Y


def _stablemax_backward(ctx, dY):
    q, k, v, qd, kd, Y = ctx.saved_tensors
    q_dt, k_dt, v_dt, qd_dt, kd_dt, cdt, scale_f, power_f = ctx.meta
    H, M, D_score = q.shape
    B, N, _, D_value = v.shape
    if M > 256 or D_score > 256 or D_value > 256:
        raise NotImplementedError(
            "The MI355X stablemax FLARE backward supports M <= 256 and head dims <= 256; "
            f"got M={M}, D_score={D_score}, D_value={D_value}."
        )
    dev = v.device
    dyc = dY.to(cdt).contiguous()
    yc = Y.to(cdt).contiguous()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dqd = torch.empty_like(qd) if qd is not None else None
    dkd = torch.empty_like(kd) if kd is not None else None
    lib = _lib.lib()
    nbytes = lib.flare_stablemax_backward_workspace_size(B, N, H, M, D_score, D_value, int(qd is not None))
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    P = _lib.ptr
    rc = lib.flare_stablemax_backward(P(q), P(k), P(v), P(qd), P(kd), _lib.dtype_code(cdt), B, N, H, M, D_score,
                                      D_value, scale_f, power_f, P(yc), P(dyc), P(dq), P(dk), P(dv), P(dqd), P(dkd),
                                      P(ws), nbytes, _lib.stream_of(dev))
    _lib.check(rc, "flare_stablemax_backward")
    # a decoder tensor that is the encoder one has its share folded into dK / dQ
    return (dq.to(q_dt), dk.to(k_dt), dv.to(v_dt), None if dqd is None else dqd.to(qd_dt),
            None if dkd is None else dkd.to(kd_dt), None, None, None, None)


class FLAREAutoregressiveStablemaxTriton(autograd.Function):
    """Stablemax FLARE forward (reference stablemax_triton.py:1707-1731)."""

    @staticmethod
    def forward(ctx, Q, K, V, Q_dec, K_dec, scale=None, chunk_size=None, power: float = 2.0, input_precision=None):
        ctx.empty_shapes = None
        if V.shape[1] == 0:
            ctx.empty_shapes = (Q, K, V, Q_dec, K_dec)
        return _stablemax_forward(Q, K, V, Q_dec, K_dec, scale, chunk_size, power, input_precision, ctx)

    @staticmethod
    def backward(ctx, dY):
        """Reference stablemax_triton.py:1981-2420 (zero gradients for an empty sequence,
        as the reference's :1982-1999)."""
        if ctx.empty_shapes is not None:
            return tuple(torch.zeros_like(t) for t in ctx.empty_shapes) + (None, None, None, None)
        return _stablemax_backward(ctx, dY)


def flare_autoregressive_stablemax_triton(
    Q,
    K,
    V,
    scale=None,
    eps=None,
    profile: bool = False,
    chunk_size=None,
    Q_dec=None,
    K_dec=None,
    power: float = 2.0,
    write_gate: bool = False,
    write_gate_fixed_value: float | None = None,
    write_gate_tensor=None,
    state: dict[str, torch.Tensor] | None = None,
    attention_mask: torch.Tensor | None = None,
    return_state: bool = False,
    input_precision=None,
):
    """Stablemax causal FLARE (reference stablemax_triton.py:2423-2468)."""
    if eps is not None:
        raise NotImplementedError("flare_autoregressive_stablemax_triton does not use eps.")
    if profile:
        raise NotImplementedError("flare_autoregressive_stablemax_triton does not support profile=True")
    if state is not None:
        raise NotImplementedError("flare_autoregressive_stablemax_triton does not support recurrent state")
    if attention_mask is not None:
        raise NotImplementedError("flare_autoregressive_stablemax_triton does not support attention_mask")
    if return_state:
        raise NotImplementedError("flare_autoregressive_stablemax_triton does not support return_state=True")
    if write_gate or write_gate_fixed_value is not None or write_gate_tensor is not None:
        raise NotImplementedError("flare_autoregressive_stablemax_triton currently implements the non-write-gated path only.")
    Q_dec_resolved, K_dec_resolved, _, _, _ = resolve_flare_causal_decode_inputs(Q, K, Q_dec, K_dec)
    return FLAREAutoregressiveStablemaxTriton.apply(
        Q, K, V, Q_dec_resolved, K_dec_resolved, scale, chunk_size, power, input_precision
    )
