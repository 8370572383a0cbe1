"""Shared host-side semantics of the causal FLARE entry points.

Each helper states the reference behaviour it keeps (path:line in
vpuri3/causal-flare).
"""
from __future__ import annotations

import torch


def _resolve_attn_scale(scale, head_dim: int) -> float:
    """Default softmax scale: 1.0 when D <= 8, else D**-0.5 (``_common.py:201-204``)."""
    if scale is not None:
        return float(scale)
    return 1.0 if head_dim <= 8 else head_dim ** -0.5


def _get_allclose_tols(dtype: torch.dtype) -> tuple[float, float]:
    """(rtol, atol): 1e-5 for fp32, 1e-2 for bf16/fp16 (``_common.py:132-137``)."""
    if dtype in (torch.float16, torch.bfloat16):
        return 1e-2, 1e-2
    return 1e-5, 1e-5


def _max_rel_err(a: torch.Tensor, b: torch.Tensor, atol: float) -> float:
    """max |a-b| / (|b| + atol) (``_common.py:144-146``)."""
    return ((a.float() - b.float()).abs() / (b.abs().float() + atol)).amax().item()


def _normalize_input_precision(input_precision) -> str:
    """Accepts the reference's precision knob (``_common.py:253-269``).

    On gfx950 the bf16/fp16 paths always use bf16/fp16 MFMA with fp32
    accumulation and the fp32 path always computes in IEEE fp32, so the value
    is validated and otherwise has no effect.
    """
    if input_precision is None:
        return "ieee"
    if isinstance(input_precision, bool):
        return "tf32" if input_precision else "ieee"
    mode = str(input_precision).strip().lower()
    if mode not in ("tf32", "tf32x3", "ieee"):
        raise ValueError(
            f"Unsupported input_precision={input_precision!r}. Expected one of {{'tf32','tf32x3','ieee'}}."
        )
    return mode


def _compute_dtype(*tensors) -> torch.dtype:
    """One element type for every input: the promotion of the given tensors' dtypes."""
    dt = None
    for t in tensors:
        if t is None:
            continue
        dt = t.dtype if dt is None else torch.promote_types(dt, t.dtype)
    if dt not in (torch.float32, torch.bfloat16, torch.float16):
        dt = torch.float32
    return dt


def _require_gpu(name: str, *tensors) -> torch.device:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"{name} requires GPU tensors (got a tensor on {t.device}).")
    return tensors[0].device


def _refresh_profile_totals(profile_data) -> None:
    """Totals in the profile dict (``training.py:41-50``)."""
    if profile_data is None:
        return
    fwd = profile_data.get("forward", {})
    bwd = profile_data.get("backward", {})
    f = float(sum(fwd.values())) if isinstance(fwd, dict) else 0.0
    b = float(sum(bwd.values())) if isinstance(bwd, dict) else 0.0
    profile_data["forward_total_ms"] = f
    profile_data["backward_total_ms"] = b
    profile_data["total_ms"] = f + b


class EventLog:
    """Per-phase GPU times of back-to-back launches: start/end events recorded on the
    launch stream with no synchronisation, read by ``mean_ms`` after the caller has
    synchronised.  Passed where a ``timings`` dict goes in the internal launchers."""

    def __init__(self):
        self.pairs = {}

    def record(self, key, op):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        out = op()
        end.record()
        self.pairs.setdefault(key, []).append((start, end))
        return out

    def mean_ms(self):
        return {k: sum(s.elapsed_time(e) for s, e in v) / len(v) for k, v in self.pairs.items()}


class _PhaseTimer:
    """Per-phase GPU time with events on the current stream (``_common.py:51-65``)."""

    def __init__(self, device, bucket):
        self.device = device
        self.bucket = bucket

    def __call__(self, key, op):
        if self.bucket is None:
            return op()
        if isinstance(self.bucket, EventLog):
            return self.bucket.record(key, op)
        torch.cuda.synchronize(self.device)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        out = op()
        end.record()
        torch.cuda.synchronize(self.device)
        self.bucket[key] = self.bucket.get(key, 0.0) + float(start.elapsed_time(end))
        return out
