"""Cached prefill and single-token decode of causal FLARE on MI355X.

Drop-ins for ``flare_autoregressive_prefill_triton`` and
``flare_autoregressive_decode_triton`` (``causal_flare/autoregressive/inference.py:492-820``):
same signatures, defaults (scale = 1.0), validation messages, state layout
``{"m": [B,H,M], "d": [B,H,M], "u": [B,H,M,Dv]}`` (fp32) and aliasing: decode
updates a contiguous fp32 state in place and returns the same tensors.
"""
from __future__ import annotations

import torch

from .. import _lib
from .._common import (
    _compute_dtype,
    _normalize_input_precision,
    _refresh_profile_totals,
    _require_gpu,
)
from .._reference_utils import resolve_flare_causal_decode_inputs
from .training import _decoder_args, _resolve_chunk_size, run_chunked_forward


def _init_flare_recurrent_state(batch_size, num_heads, num_latents, value_head_dim, device,
                                dtype=torch.float32):
    """Fresh state: m = -inf, d = 0, u = 0 (reference inference.py:66-84)."""
    return {
        "m": torch.full((batch_size, num_heads, num_latents), -torch.inf, device=device, dtype=dtype),
        "d": torch.zeros((batch_size, num_heads, num_latents), device=device, dtype=dtype),
        "u": torch.zeros((batch_size, num_heads, num_latents, value_head_dim), device=device, dtype=dtype),
    }


def _canonicalize_flare_state(state, batch_size, num_heads, num_latents, value_head_dim, device):
    """fp32 state on `device` with shape checks (reference inference.py:86-120).

    ``.to()`` returns the caller's tensors unchanged when they are already fp32
    on the device, which is what lets decode update the state in place.
    """
    if state is None:
        return _init_flare_recurrent_state(batch_size, num_heads, num_latents, value_head_dim, device)
    if not isinstance(state, dict):
        raise ValueError(f"FLARE recurrent state must be a dict with keys {'m', 'd', 'u'}. Got {type(state)}")
    if not all(k in state for k in ("m", "d", "u")):
        raise ValueError(f"Invalid FLARE recurrent state keys: {list(state.keys())}")
    m = state["m"].to(device=device, dtype=torch.float32)
    d = state["d"].to(device=device, dtype=torch.float32)
    u = state["u"].to(device=device, dtype=torch.float32)
    es = (batch_size, num_heads, num_latents)
    eu = (batch_size, num_heads, num_latents, value_head_dim)
    if tuple(m.shape) != es or tuple(d.shape) != es or tuple(u.shape) != eu:
        raise ValueError(
            "Invalid FLARE recurrent state shapes. "
            f"Expected m/d={es}, u={eu}; "
            f"got m={tuple(m.shape)}, d={tuple(d.shape)}, u={tuple(u.shape)}"
        )
    return {"m": m, "d": d, "u": u}


def _canonicalize_kv_for_prefill(K, V):
    if K.dim() != 4 or V.dim() != 4:
        raise ValueError(f"Prefill expects K/V to be [B, T, H, D]. Got K={tuple(K.shape)}, V={tuple(V.shape)}")
    if K.shape[:3] != V.shape[:3]:
        raise ValueError(
            f"Prefill expects K and V to agree on [B, T, H]. Got K={tuple(K.shape)}, V={tuple(V.shape)}"
        )
    return K, V


def _canonicalize_kv_for_decode(K, V):
    if K.dim() == 4 and K.shape[1] == 1:
        K = K[:, 0]
    if V.dim() == 4 and V.shape[1] == 1:
        V = V[:, 0]
    if K.dim() != 3 or V.dim() != 3:
        raise ValueError(f"Decode expects K/V as [B, H, D] or [B, 1, H, D]. Got K={tuple(K.shape)}, V={tuple(V.shape)}")
    if K.shape[:2] != V.shape[:2]:
        raise ValueError(
            f"Decode expects K and V to agree on [B, H]. Got K={tuple(K.shape)}, V={tuple(V.shape)}"
        )
    return K, V


def _canonicalize_q_dec_for_decode(Q_dec, K_step, K_input=None, K_prefill=None):
    """Decode-step decoder query as [B, 1, H, D] (reference inference.py:155-191)."""
    if Q_dec is None:
        return None
    if Q_dec is K_step or (K_input is not None and Q_dec is K_input):
        return K_prefill if K_prefill is not None else K_step[:, None, :, :]
    if Q_dec.dim() == 3:
        if Q_dec.shape != K_step.shape:
            raise ValueError(
                "Decode Q_dec must match K decode-step shape. "
                f"Got Q_dec.shape={tuple(Q_dec.shape)} and K.shape={tuple(K_step.shape)}"
            )
        return Q_dec[:, None, :, :]
    if Q_dec.dim() == 4:
        if Q_dec.shape[0] != K_step.shape[0] or Q_dec.shape[2] != K_step.shape[1] or Q_dec.shape[3] != K_step.shape[2]:
            raise ValueError(
                "Decode Q_dec [B, 1, H, D] must match K [B, H, D]. "
                f"Got Q_dec.shape={tuple(Q_dec.shape)} and K.shape={tuple(K_step.shape)}"
            )
        if Q_dec.shape[1] != 1:
            raise ValueError(
                f"Decode Q_dec with rank-4 must have sequence length 1. Got Q_dec.shape={tuple(Q_dec.shape)}"
            )
        return Q_dec
    raise ValueError(f"Decode Q_dec must be [B, H, D] or [B, 1, H, D]. Got Q_dec.shape={tuple(Q_dec.shape)}")


def _decode_step_fast(Q, K, V, state, scale):
    """The common decode call, with the host work cut to the launch itself: shared
    decoder weights, no mask, Q/K/V of one 16-bit or fp32 type and contiguous, and
    a contiguous fp32 state on the same device.  Returns None (the general path
    then runs, with its full validation) when any of that does not hold."""
    if K.dim() == 4:
        if K.shape[1] != 1:
            return None
        B, _, H, Dk = K.shape
    elif K.dim() == 3:
        B, H, Dk = K.shape
    else:
        return None
    if V.dim() not in (3, 4) or (V.dim() == 4 and V.shape[1] != 1) or Q.dim() != 3:
        return None
    Dv = V.shape[-1]
    Hq, M, Dq = Q.shape
    dt = Q.dtype
    if (Hq != H or Dq != Dk or V.shape[0] != B or V.shape[-2] != H or K.dtype is not dt or V.dtype is not dt
            or dt not in _FAST_DTYPES or not (Q.is_contiguous() and K.is_contiguous() and V.is_contiguous())):
        return None
    if not isinstance(state, dict):
        return None
    m, d, u = state.get("m"), state.get("d"), state.get("u")
    dev = K.device
    for t in (m, d, u):
        if (t is None or t.dtype is not torch.float32 or t.device != dev or not t.is_contiguous()):
            return None
    if m.shape != (B, H, M) or d.shape != (B, H, M) or u.shape != (B, H, M, Dv) or u.data_ptr() % 16:
        return None
    if V.device != dev or Q.device != dev:
        return None
    y = torch.empty((B, 1, H, Dv), device=dev, dtype=dt)
    code = _FAST_DTYPES[dt]
    rc = _lib.lib().flare_decode_step(Q.data_ptr(), K.data_ptr(), V.data_ptr(), None, None, None, code, B, H, M,
                                      Dk, Dv, float(scale), m.data_ptr(), d.data_ptr(), u.data_ptr(), y.data_ptr(),
                                      code, _raw_stream(dev.index))
    _lib.check(rc, "flare_decode_step")
    return y, {"m": m, "d": d, "u": u}


_FAST_DTYPES = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}


def _raw_stream(index):
    """Handle of the current stream of device `index` (None: the current device)."""
    if index is None:
        index = torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def flare_autoregressive_decode_triton(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    state: dict[str, torch.Tensor] | None = None,
    scale: float = 1.0,
    input_precision: str | None = None,
    attention_mask: torch.Tensor | None = None,
    Q_dec: torch.Tensor | None = None,
    K_dec: torch.Tensor | None = None,
    profile: bool = False,
):
    """One recurrent decode step (reference inference.py:492-621); one kernel launch."""
    if Q.device.type != "cuda":
        raise RuntimeError("flare_autoregressive_decode requires CUDA tensors. ")
    if (Q_dec is None and K_dec is None and attention_mask is None and input_precision is None
            and not profile and state is not None):
        out = _decode_step_fast(Q, K, V, state, scale)
        if out is not None:
            return out
    K_input = K
    K, V = _canonicalize_kv_for_decode(K, V)
    _normalize_input_precision(input_precision)
    B, H, D_score = K.shape
    D_value = V.shape[-1]
    Hq, M, Dq = Q.shape
    if Hq != H or Dq != D_score:
        raise ValueError(f"Incompatible Q/K shapes. Q={tuple(Q.shape)}, K={tuple(K.shape)}")
    K_resolve = K[:, None, :, :]
    Q_dec_resolve = _canonicalize_q_dec_for_decode(Q_dec, K, K_input=K_input, K_prefill=K_resolve)
    Q_dec_resolve, K_dec_resolve, sep_q, sep_k, shared = resolve_flare_causal_decode_inputs(
        Q, K_resolve, Q_dec_resolve, K_dec
    )
    mask = None
    if attention_mask is not None:
        if attention_mask.dim() == 2 and attention_mask.shape[1] == 1:
            attention_mask = attention_mask[:, 0]
        if attention_mask.dim() != 1 or attention_mask.shape[0] != B:
            raise ValueError(f"Decode attention_mask must be [B] or [B, 1]. Got {tuple(attention_mask.shape)}")
        mask = attention_mask.to(device=K.device, dtype=torch.int32).contiguous()

    st = _canonicalize_flare_state(state, B, H, M, D_value, K.device)
    m_state = st["m"].contiguous()
    d_state = st["d"].contiguous()
    u_state = st["u"].contiguous()

    qd = kd = None
    if not shared:
        if sep_q and Q_dec_resolve is not K_resolve:
            qd = Q_dec_resolve[:, 0]
        if sep_k and K_dec_resolve is not Q:
            kd = K_dec_resolve
    cdt = _compute_dtype(Q, K, V, qd, kd)
    q, k, v = (t if (t.dtype == cdt and t.is_contiguous()) else t.to(cdt).contiguous() for t in (Q, K, V))
    qd = None if qd is None else qd.to(cdt).contiguous()
    kd = None if kd is None else kd.to(cdt).contiguous()
    y = torch.empty((B, H, D_value), device=K.device, dtype=V.dtype)
    # The kernel streams u with 16-byte accesses; a misaligned view runs on an
    # aligned copy that is written back, so the caller's tensor is still updated.
    u_run = u_state if u_state.data_ptr() % 16 == 0 else u_state.clone()
    P = _lib.ptr
    lib = _lib.lib()
    launch = lambda: lib.flare_decode_step(
        P(q), P(k), P(v), P(qd), P(kd), P(mask), _lib.dtype_code(cdt), B, H, M, D_score, D_value,
        float(scale), P(m_state), P(d_state), P(u_run), P(y), _lib.dtype_code(V.dtype),
        _lib.stream_of(K.device))
    profile_data = None
    if profile:
        from .._common import _PhaseTimer
        profile_data = {"forward": {}}
        rc = _PhaseTimer(K.device, profile_data["forward"])("flare_autoregressive_decode_step", launch)
    else:
        rc = launch()
    _lib.check(rc, "flare_decode_step")
    if u_run is not u_state:
        u_state.copy_(u_run)
    next_state = {"m": m_state, "d": d_state, "u": u_state}
    y_out = y[:, None, :, :]
    if profile:
        _refresh_profile_totals(profile_data)
        return (y_out, next_state), profile_data
    return y_out, next_state


def flare_autoregressive_prefill_triton(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    state: dict[str, torch.Tensor] | None = None,
    scale: float = 1.0,
    input_precision: str | None = None,
    attention_mask: torch.Tensor | None = None,
    Q_dec: torch.Tensor | None = None,
    K_dec: torch.Tensor | None = None,
    profile: bool = False,
):
    """Cached prefill (reference inference.py:624-820): returns (Y [B,T,H,Dv] in V.dtype, final state)."""
    if Q.device.type != "cuda":
        raise RuntimeError("flare_autoregressive_prefill requires CUDA tensors.")
    K, V = _canonicalize_kv_for_prefill(K, V)
    B, T, H, D_score = K.shape
    D_value = V.shape[-1]
    if Q.dim() != 3:
        raise ValueError(f"Q must be [H, M, D]. Got Q={tuple(Q.shape)}")
    Hq, M, Dq = Q.shape
    if Hq != H or Dq != D_score:
        raise ValueError(f"Incompatible Q/K shapes. Q={tuple(Q.shape)}, K={tuple(K.shape)}")
    if attention_mask is not None and attention_mask.shape != (B, T):
        raise ValueError(f"attention_mask must be [B, T]. Got {tuple(attention_mask.shape)}")
    Q_dec, K_dec, sep_q, sep_k, shared = resolve_flare_causal_decode_inputs(Q, K, Q_dec, K_dec)
    _normalize_input_precision(input_precision)
    if T == 0:
        st = _canonicalize_flare_state(state, B, H, M, D_value, K.device)
        return torch.empty((B, 0, H, D_value), device=K.device, dtype=V.dtype), st

    token_mask = None
    if attention_mask is not None:
        # The reference runs a masked prefill as the decode step token by token
        # (inference.py:663-695): a masked token leaves the state unchanged and gets
        # y = 0.  The chunked kernels apply the same rule to the whole sequence.
        if not bool((attention_mask != 0).all().item()):
            token_mask = (attention_mask != 0).to(device=K.device, dtype=torch.int32).contiguous()

    _require_gpu("flare_autoregressive_prefill", Q, K, V)
    st = None if state is None else _canonicalize_flare_state(state, B, H, M, D_value, K.device)
    if st is not None:   # contiguous and 16-byte aligned (the scan reads u with 16-byte loads)
        st = {k: (v.contiguous() if v.data_ptr() % 16 == 0 else v.contiguous().clone()) for k, v in st.items()}
    _, chunk = _resolve_chunk_size(None, B, T, H, M, D_value)
    qd, kd = (None, None) if shared else _decoder_args(Q, K, Q_dec, K_dec, sep_q, sep_k)
    profile_data = {"forward": {}} if profile else None
    Y, next_state = run_chunked_forward(
        Q, K, V, qd, kd, scale=float(scale), chunk=chunk, out_dtype=V.dtype, state=st,
        want_state=True, timings=profile_data["forward"] if profile else None, token_mask=token_mask,
    )
    if profile:
        _refresh_profile_totals(profile_data)
        return (Y, next_state), profile_data
    return Y, next_state


def flare_prefill(Q, K, V, state=None, scale=1.0, input_precision=None, attention_mask=None,
                  impl="triton", Q_dec=None, K_dec=None):
    """Dispatcher (reference inference.py:823-858); only the GPU implementation exists here."""
    if impl != "triton":
        raise ValueError(f"Unsupported impl={impl}. This build provides only impl='triton' (the HIP kernels).")
    return flare_autoregressive_prefill_triton(Q=Q, K=K, V=V, Q_dec=Q_dec, K_dec=K_dec, state=state,
                                               scale=scale, input_precision=input_precision,
                                               attention_mask=attention_mask)


def flare_decode(Q, K, V, state, scale=1.0, input_precision=None, attention_mask=None,
                 impl="triton", Q_dec=None, K_dec=None):
    """Dispatcher (reference inference.py:861-896); only the GPU implementation exists here."""
    if impl != "triton":
        raise ValueError(f"Unsupported impl={impl}. This build provides only impl='triton' (the HIP kernels).")
    return flare_autoregressive_decode_triton(Q=Q, K=K, V=V, state=state, Q_dec=Q_dec, K_dec=K_dec,
                                              scale=scale, input_precision=input_precision,
                                              attention_mask=attention_mask)
