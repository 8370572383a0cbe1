"""Helpers shared by the tests: seeded inputs and the tolerance checks."""
import numpy as np
import torch


def seeded(seed, B, N, H, M, Dk, Dv, dtype, q_std=1.0, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn((H, M, Dk), generator=g) * q_std).to(dtype)
    k = torch.randn((B, N, H, Dk), generator=g).to(dtype)
    v = torch.randn((B, N, H, Dv), generator=g).to(dtype)
    return q.to(device), k.to(device), v.to(device)


def max_rel_err(a, b, atol):
    """max |a-b| / (|b| + atol): the reference's _max_rel_err (_common.py:144-146)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if a.size == 0:
        return 0.0
    return float((np.abs(a - b) / (np.abs(b) + atol)).max())


def to_np(t):
    return t.detach().float().cpu().numpy() if hasattr(t, "detach") else np.asarray(t)


# Tolerances (stated once, used by every GPU parity test):
#   bf16 / fp16 inputs: max_rel_err(atol=1e-2) <= 1e-2 against the fp32 oracle
#                       (north star; atol from _common.py:132-137).
#   fp32 inputs:        |a-b| <= 1e-5 + 1e-4*|b|, the reference's own fp32
#                       parity bar (testing/autoregressive/test_flare.py:367).
#                       max_rel_err(atol=1e-5) itself is not bounded for fp32:
#                       entries that cancel to ~1e-4 carry ~1e-7 absolute
#                       rounding from a different summation order, so the
#                       quotient reaches ~1e-2 for any two fp32 implementations.
def assert_parity(out, ref, dtype, what=""):
    a, b = to_np(out), to_np(ref)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite output"
    if dtype in (torch.bfloat16, torch.float16):
        err = max_rel_err(a, b, 1e-2)
        assert err <= 1e-2, f"{what}: bf16 max_rel_err {err:.3e} > 1e-2"
    else:
        diff = np.abs(a - b)
        bound = 1e-5 + 1e-4 * np.abs(b)
        worst = float((diff - bound).max()) if diff.size else 0.0
        assert worst <= 0, f"{what}: fp32 max abs diff {diff.max():.3e} exceeds 1e-5 + 1e-4|ref|"
    return max_rel_err(a, b, 1e-2 if dtype != torch.float32 else 1e-5)
