"""Full-sequence chunked causal FLARE forward on MI355X.

Drop-in for ``flare_autoregressive_triton`` / ``AutoRegressiveFLARE``
(``causal_flare/autoregressive/training.py:731-905, 4921-4932``): same
signature, defaults, assertions and return arity.  The three phases run as
HIP kernels from ``libflare_mi355x.so``:

    flare_chunk_prepare -> flare_chunk_prefix -> flare_chunk_output

(reference kernels flare_chunk_prepare :914, flare_chunk_prefix :1021,
flare_chunk_decoder_lse :1106 + flare_chunk_fwd :1189).

The backward pass (reference ``_chunked_flare_lse_backward_impl``,
training.py:4369-4918) runs as HIP kernels through ``flare_ar_backward``; it
recomputes the chunk statistics from the saved inputs and output.
"""
from __future__ import annotations

import ctypes
import os

import torch
import torch.autograd as autograd

from .. import _lib
from .._common import (
    _PhaseTimer,
    _compute_dtype,
    _normalize_input_precision,
    _refresh_profile_totals,
    _require_gpu,
    _resolve_attn_scale,
)
from .._reference_utils import resolve_flare_causal_decode_inputs


def _resolve_chunk_size(chunk_size, B, N, H, M, Dv, validate_only=False) -> tuple[int, int]:
    """(validated chunk_size, kernel chunk length).

    The reference's default chunk is 64 (training.py:328-337) and must be a
    multiple of 16 (:344).  Chunk length only changes fp32 rounding, so when
    neither ``chunk_size`` nor FLARE_CHUNK_SIZE is given the library's own
    policy (about one chunk workgroup per compute unit) is used.
    """
    explicit = chunk_size
    if explicit is None:
        env = os.environ.get("FLARE_CHUNK_SIZE", "")
        explicit = int(env) if env else None
    requested = 64 if explicit is None else int(explicit)
    assert requested % 16 == 0, f"CHUNK_SIZE must be divisible by 16. Got CHUNK_SIZE={requested}."
    if validate_only:
        return requested, requested
    if explicit is None:
        return requested, int(_lib.lib().flare_ar_default_chunk(B, N, H, M, Dv))
    return requested, requested


def _decoder_args(Q, K, Q_dec, K_dec, separate_q, separate_k):
    """C-ABI decoder pointers: None selects the encoder tensor (K for Q_dec, Q for K_dec)."""
    qd = Q_dec if (separate_q and Q_dec is not K) else None
    kd = K_dec if (separate_k and K_dec is not Q) else None
    return qd, kd


def _prep(t, dtype):
    return None if t is None else t.to(dtype).contiguous()


_PHASES = ("flare_chunk_prepare", "flare_chunk_prefix", "flare_chunk_fwd")


def forward_kernel_resources(dtype, M, Dk, Dv, shared, chunk):
    """Per phase, the resources of the kernel the forward launches: waves per workgroup,
    VGPRs per lane, spilled 4-byte slots per lane and LDS bytes per workgroup (the
    reference's _maybe_record_kernel_resource, training.py:4-18, reads the same facts
    from Triton's compiled kernels).  A phase whose kernel the library does not report
    (scalar or earlier kernels) is left out."""
    lib = _lib.lib()
    out = (ctypes.c_int32 * 4)()
    res = {}
    for phase, name in enumerate(_PHASES):
        rc = lib.flare_forward_kernel_resources(_lib.dtype_code(dtype), M, Dk, Dv, int(shared), chunk, phase,
                                                ctypes.cast(out, ctypes.c_void_p))
        if rc != 0:
            continue
        res[name] = {"num_waves": int(out[0]), "regs_per_thread": int(out[1]), "spills": int(out[2]) // 4,
                     "shared_bytes": int(out[3])}
    return res


def run_chunked_forward(Q, K, V, qd, kd, *, scale, chunk, out_dtype, state=None,
                        want_state=False, timings=None, token_mask=None):
    """Launch phases 1-3; returns (Y, final_state or None).  Inputs are validated by the caller.

    token_mask: optional int32 [B, N] (nonzero = keep); a masked token adds nothing
    to the state and gets y = 0."""
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    device = K.device
    cdt = _compute_dtype(Q, K, V, qd, kd)
    code = _lib.dtype_code(cdt)
    q, k, v, qd, kd = (_prep(t, cdt) for t in (Q, K, V, qd, kd))
    lib = _lib.lib()
    stream = _lib.stream_of(device)
    Y = torch.empty((B, N, H, Dv), device=device, dtype=out_dtype)
    out_code = _lib.dtype_code(out_dtype)
    m0 = d0 = u0 = None
    if state is not None:
        m0, d0, u0 = state["m"], state["d"], state["u"]
    fin = None
    if want_state:
        fin = {
            "m": torch.empty((B, H, M), device=device, dtype=torch.float32),
            "d": torch.empty((B, H, M), device=device, dtype=torch.float32),
            "u": torch.empty((B, H, M, Dv), device=device, dtype=torch.float32),
        }
    P = _lib.ptr
    fin_ptrs = (P(fin["m"]), P(fin["d"]), P(fin["u"])) if fin else (None, None, None)
    NC = (N + chunk - 1) // chunk
    if timings is None or token_mask is not None:
        size_fn = (lib.flare_ar_forward_workspace_size if qd is None and kd is None
                   else lib.flare_ar_forward_workspace_size_sep)
        nbytes = size_fn(B, N, H, M, Dv, chunk)
        ws = torch.empty(nbytes, device=device, dtype=torch.uint8)
        if token_mask is None:
            rc = lib.flare_ar_forward(P(q), P(k), P(v), P(qd), P(kd), code, B, N, H, M, Dk, Dv,
                                      float(scale), chunk, P(m0), P(d0), P(u0), *fin_ptrs, P(Y),
                                      out_code, P(ws), nbytes, stream)
            _lib.check(rc, "flare_ar_forward")
        else:
            tm = token_mask.to(device=device, dtype=torch.int32).contiguous()
            rc = lib.flare_ar_forward_masked(P(q), P(k), P(v), P(qd), P(kd), code, B, N, H, M, Dk, Dv,
                                             float(scale), chunk, P(m0), P(d0), P(u0), *fin_ptrs, P(Y),
                                             out_code, P(tm), P(ws), nbytes, stream)
            _lib.check(rc, "flare_ar_forward_masked")
        return Y, fin
    timer = _PhaseTimer(device, timings)
    cmax = torch.empty((B * H, NC, M), device=device, dtype=torch.float32)
    cden = torch.empty_like(cmax)
    cnum = torch.empty((B * H, NC, M, Dv), device=device, dtype=torch.float32)
    _lib.check(timer("flare_chunk_prepare", lambda: lib.flare_chunk_prepare(
        P(q), P(k), P(v), code, B, N, H, M, Dk, Dv, float(scale), chunk, P(cmax), P(cden),
        P(cnum), stream)), "flare_chunk_prepare")
    _lib.check(timer("flare_chunk_prefix", lambda: lib.flare_chunk_prefix(
        P(cmax), P(cden), P(cnum), B * H, NC, M, Dv, P(m0), P(d0), P(u0), *fin_ptrs, stream)),
        "flare_chunk_prefix")
    _lib.check(timer("flare_chunk_fwd", lambda: lib.flare_chunk_output(
        P(q), P(k), P(v), P(qd), P(kd), code, B, N, H, M, Dk, Dv, float(scale), chunk, P(cmax),
        P(cden), P(cnum), P(Y), out_code, None, stream)), "flare_chunk_fwd")
    return Y, fin


def run_chunked_backward(Q, K, V, qd, kd, Y, dY, *, scale):
    """Launch flare_ar_backward; returns (dQ, dK, dV, dQ_dec, dK_dec) in the
    inputs' dtypes (None for a decoder tensor that was not separate)."""
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    if dY is None:
        return None, None, None, None, None
    if N == 0:
        return tuple(None if t is None else torch.zeros_like(t) for t in (Q, K, V, qd, kd))
    if M > 256 or Dk > 256 or Dv > 512:
        raise NotImplementedError(
            f"The MI355X FLARE backward supports M <= 256, D_score <= 256 and D_value <= 512; "
            f"got M={M}, D_score={Dk}, D_value={Dv}."
        )
    device = K.device
    cdt = _compute_dtype(Q, K, V, qd, kd)
    code = _lib.dtype_code(cdt)
    q, k, v, qdc, kdc, y, dy = (_prep(t, cdt) for t in (Q, K, V, qd, kd, Y, dY))
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dqd = torch.empty_like(qdc) if qdc is not None else None
    dkd = torch.empty_like(kdc) if kdc is not None else None
    lib = _lib.lib()
    nbytes = lib.flare_ar_backward_workspace_size(B, N, H, M, Dk, Dv)
    ws = torch.empty(nbytes, device=device, dtype=torch.uint8)
    P = _lib.ptr
    rc = lib.flare_ar_backward(P(q), P(k), P(v), P(qdc), P(kdc), code, B, N, H, M, Dk, Dv, float(scale),
                               P(y), P(dy), P(dq), P(dk), P(dv), P(dqd), P(dkd), P(ws), nbytes,
                               _lib.stream_of(device))
    _lib.check(rc, "flare_ar_backward")
    cast = lambda g, ref: None if g is None else g.to(ref.dtype)
    return cast(dq, Q), cast(dk, K), cast(dv, V), cast(dqd, qd), cast(dkd, kd)


class AutoRegressiveFLARE(autograd.Function):
    """Forward of causal FLARE (reference ``training.py:731-905``)."""

    @staticmethod
    def forward(ctx, Q, K, V, scale=None, chunk_size=None, input_precision=None, profile=False,
                Q_dec=None, K_dec=None):
        assert Q.dim() == 3 and K.dim() == 4 and V.dim() == 4, (
            "Q, K, V must be 3D and 4D tensors respectively "
            f"got Q.dim()={Q.dim()}, K.dim()={K.dim()}, V.dim()={V.dim()}"
        )
        assert K.shape[:3] == V.shape[:3], (
            f"Expected K/V to agree on [B, N, H]. Got K.shape={K.shape} and V.shape={V.shape}"
        )
        assert Q.size(0) == K.size(2) and Q.size(2) == K.size(3), (
            f"Expected Q [H, M, D_k] and K [B, N, H, D_k]. Got Q.shape={Q.shape} and K.shape={K.shape}"
        )
        H, M, D_score = Q.shape
        B, N, _, D_value = V.shape
        Q_dec_r, K_dec_r, sep_q, sep_k, shared = resolve_flare_causal_decode_inputs(Q, K, Q_dec, K_dec)
        scale = _resolve_attn_scale(scale, D_score)
        _normalize_input_precision(input_precision)
        assert M % 16 == 0, f"M must be divisible by 16. Got M={M}."
        assert D_score % 16 == 0, f"score_head_dim must be divisible by 16. Got score_head_dim={D_score}."
        assert D_value % 16 == 0, f"value_head_dim must be divisible by 16. Got value_head_dim={D_value}."
        _resolve_chunk_size(chunk_size, B, N, H, M, D_value, validate_only=True)
        _require_gpu("flare_autoregressive_triton", Q, K, V, Q_dec, K_dec)
        # Output in the compute dtype of K (training.py:322-324, 724-727).
        out_dtype = K.dtype if K.dtype in (torch.bfloat16, torch.float16) else torch.float32
        profile_data = {"forward": {}, "backward": {}} if profile else None
        qd = kd = None
        if N == 0:
            Y = torch.empty((B, 0, H, D_value), device=K.device, dtype=out_dtype)
        else:
            _, chunk = _resolve_chunk_size(chunk_size, B, N, H, M, D_value)
            qd, kd = (None, None) if shared else _decoder_args(Q, K, Q_dec_r, K_dec_r, sep_q, sep_k)
            Y, _ = run_chunked_forward(
                Q, K, V, qd, kd, scale=scale, chunk=chunk, out_dtype=out_dtype,
                timings=profile_data["forward"] if profile else None,
            )
            if profile:
                profile_data["forward_resources"] = forward_kernel_resources(
                    _compute_dtype(Q, K, V, qd, kd), M, D_score, D_value, qd is None and kd is None, chunk)
        ctx.scale = scale
        ctx.sep = (qd is not None, kd is not None)
        ctx.save_for_backward(Q, K, V, qd, kd, Y)
        if profile:
            _refresh_profile_totals(profile_data)
            return Y, profile_data
        return Y

    @staticmethod
    def backward(ctx, dY, *_unused):
        """Gradients of Q, K, V (and Q_dec, K_dec when separate): reference
        _chunked_flare_lse_backward_impl (training.py:4369-4918)."""
        Q, K, V, qd, kd, Y = ctx.saved_tensors
        grads = run_chunked_backward(Q, K, V, qd, kd, Y, dY, scale=ctx.scale)
        return (*grads[:3], None, None, None, None, *grads[3:])


def flare_autoregressive_triton(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    scale: float | None = None,
    chunk_size: int | None = None,
    input_precision: str | None = None,
    profile: bool = False,
    Q_dec: torch.Tensor | None = None,
    K_dec: torch.Tensor | None = None,
):
    """Causal FLARE forward. Q [H,M,D], K/V [B,N,H,D] -> Y [B,N,H,D] (reference training.py:4921)."""
    return AutoRegressiveFLARE.apply(Q, K, V, scale, chunk_size, input_precision, profile, Q_dec, K_dec)


# Names the reference keeps for downstream callers (training.py:4935-4937).
ChunkedFLARE = AutoRegressiveFLARE
flare_chunk_triton = flare_autoregressive_triton
