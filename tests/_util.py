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


def assert_state_parity(st, ref, dtype, what=""):
    """Cached state {m, d, u} against the oracle.

    m and d are compared directly (fp32 bar for fp32 inputs, rtol 1e-3 for
    bf16).  For bf16 inputs u, an unnormalised sum over every token, is
    compared through z = u / d, the quantity the readout uses, with the bf16
    output bar; for fp32 inputs u is compared directly.
    """
    m, d, u = (to_np(st[k]) for k in ("m", "d", "u"))
    mr, dr, ur = (np.asarray(ref[k], np.float64) for k in ("m", "d", "u"))
    if dtype == torch.float32:
        for a, b, k in ((m, mr, "m"), (d, dr, "d"), (u, ur, "u")):
            assert_parity(a, b, torch.float32, f"{what} state {k}")
        return
    assert np.allclose(m, mr, rtol=1e-4, atol=1e-4), f"{what}: state m differs by {np.abs(m - mr).max():.3e}"
    assert np.allclose(d, dr, rtol=1e-3, atol=1e-6), f"{what}: state d differs by {(np.abs(d - dr) / np.abs(dr)).max():.3e}"
    assert_parity(u / d[..., None], ur / dr[..., None], dtype, f"{what} state z = u/d")


def assert_noise_model(out, ref, what=""):
    """bf16 check for sharp softmaxes, after the reference's suite policy
    (testing/suite_runners/correctness.py:52-59, 103-113): max-abs <= 3e-2, and
    the mean-abs error may exceed the error of rounding the fp32 reference
    itself to bf16 by at most 3e-4."""
    a, b = to_np(out).astype(np.float64), np.asarray(ref, np.float64)
    floor = float(np.abs(torch.tensor(b).to(torch.bfloat16).double().numpy() - b).mean())
    d = np.abs(a - b)
    assert np.isfinite(a).all(), f"{what}: non-finite output"
    assert d.max() <= 3e-2, f"{what}: max-abs {d.max():.3e} > 3e-2"
    assert d.mean() <= floor + 3e-4, f"{what}: mean-abs {d.mean():.3e} > bf16 floor {floor:.3e} + 3e-4"


def assert_state_rowwise(got, ref, dtype, what=""):
    """A state or chunk summary (max, den, num) against the fp64 oracle, row by row.

      max:  |m - m_ref| <= 1e-5 (natural-log units; -inf where the oracle has it)
      den:  |d - d_ref| <= 1e-5 d_ref
      num:  through z = num / den per row (one latent's D_v vector):
            max_j |z_j - zref_j| <= tol max_j |zref_j|, tol 2e-3 for bf16 / fp16
            inputs (half a bf16 ulp), 2e-5 for fp32 inputs.
    A sum over few tokens is dominated by a few of them, so single entries of z cancel
    to near zero while the row's scale is set by the large terms; the element-wise bar
    of assert_state_parity would then measure that cancellation (fp16 E in the MFMA
    paths rounds each term to 2^-11), not the kernel.
    """
    m, d, u = (to_np(t) for t in got)
    mr, dr, ur = (np.asarray(t, np.float64) for t in ref)
    assert np.isfinite(d).all() and np.isfinite(u).all(), f"{what}: non-finite"
    fin = np.isfinite(mr)
    assert (np.isneginf(m) == ~fin).all(), f"{what}: empty-row pattern differs"
    assert np.abs(m[fin] - mr[fin]).max(initial=0) <= 1e-5, f"{what}: max err {np.abs(m[fin] - mr[fin]).max()}"
    assert (np.abs(d - dr) <= 1e-5 * dr + 1e-30).all(), f"{what}: den rel err {(np.abs(d - dr) / dr).max()}"
    pos = dr > 0
    z, zr = u[pos] / d[pos][..., None], ur[pos] / dr[pos][..., None]
    tol = 2e-5 if dtype == torch.float32 else 2e-3
    err = (np.abs(z - zr).max(-1) / np.abs(zr).max(-1).clip(1e-30)).max(initial=0)
    assert err <= tol, f"{what}: z row-norm-wise err {err:.3e} > {tol}"
    return err
