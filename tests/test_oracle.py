"""Pins for the CPU oracle (oracle/flare_oracle.c and oracle/flare_oracle.py).

The reference holds no golden vectors (all of its tests draw torch.randn at run
time), so the C restatement is pinned by
  * the fp64 brute-force definitions the reference itself treats as ground
    truth (reference.py:15-47, semi_autoregressive/reference.py:560-597),
  * torch's scaled_dot_product_attention for the special cases that reduce to
    textbook attention (M = 1; semi-AR with block = N),
  * invariants (chunk-size independence, prefill/decode continuation, state
    continuation, masked tokens, semi-AR vs AR at block ends) and closed
    forms (N = 1, constant V),
  * the committed fixtures in tests/golden/ (written by
    tests/golden/make_golden.py from the fp64 definitions).
Each check is chosen so that a plausible slip in the oracle -- a dropped
prefix term, a wrong max in a rescale, a transposed operand, a missing scale
-- fails at least one of them.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import flare_oracle as O
from _util import seeded

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _close(a, b, tol=2e-5):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape
    np.testing.assert_allclose(a, b, rtol=tol, atol=tol)


@pytest.mark.parametrize("B,N,H,M,Dk,Dv", [(1, 7, 2, 16, 16, 16), (2, 37, 3, 8, 8, 24), (1, 70, 1, 32, 64, 32)])
@pytest.mark.parametrize("chunk", [1, 5, 16, 64, None])
def test_chunked_matches_brute_force(B, N, H, M, Dk, Dv, chunk):
    q, k, v = seeded(1, B, N, H, M, Dk, Dv, torch.float32)
    y = O.ar_chunked(q, k, v, chunk_size=chunk)
    _close(y, O.brute_ar(q, k, v))


@pytest.mark.parametrize("sep_q,sep_k", [(False, True), (True, False), (True, True)])
def test_chunked_separate_decoder_matches_brute_force(sep_q, sep_k):
    B, N, H, M, D = 2, 29, 2, 16, 16
    q, k, v = seeded(2, B, N, H, M, D, D, torch.float32)
    g = torch.Generator().manual_seed(5)
    qd = torch.randn(k.shape, generator=g) if sep_q else None
    kd = torch.randn(q.shape, generator=g) if sep_k else None
    y = O.ar_chunked(q, k, v, chunk_size=8, Q_dec=qd, K_dec=kd)
    _close(y, O.brute_ar(q, k, v, Q_dec=qd, K_dec=kd))
    # the decoder really is used: the result differs from the shared-weight one
    assert np.abs(y - O.ar_chunked(q, k, v, chunk_size=8)).max() > 1e-3


def test_scale_default_and_explicit():
    q, k, v = seeded(3, 1, 20, 2, 16, 32, 32, torch.float32)
    _close(O.ar_chunked(q, k, v), O.ar_chunked(q, k, v, scale=32 ** -0.5))
    assert np.abs(O.ar_chunked(q, k, v, scale=1.0) - O.ar_chunked(q, k, v)).max() > 1e-3
    _close(O.ar_chunked(q, k, v, scale=0.7), O.brute_ar(q, k, v, scale=0.7))
    assert O.resolve_scale(None, 8) == 1.0 and O.resolve_scale(None, 16) == 0.25


def test_recurrent_matches_brute_force_and_chunked():
    B, T, H, M, D = 2, 33, 2, 16, 24
    q, k, v = seeded(4, B, T, H, M, D, D, torch.float32)
    y, st = O.ar_recurrent(q, k, v, scale=0.3)
    yb, stb = O.brute_ar_state(q, k, v, scale=0.3)
    _close(y, yb)
    for key in ("m", "d", "u"):
        _close(st[key], stb[key], 1e-4)
    yc, stc = O.ar_chunked(q, k, v, scale=0.3, chunk_size=7, return_state=True)
    _close(yc, y)
    for key in ("m", "d", "u"):
        _close(stc[key], st[key], 1e-4)


def test_prefill_then_decode_equals_longer_prefill():
    B, T, H, M, D = 2, 20, 2, 16, 16
    q, k, v = seeded(6, B, T + 3, H, M, D, D, torch.float32)
    y_all, st_all = O.ar_recurrent(q, k, v)
    y, st = O.ar_recurrent(q, k[:, :T], v[:, :T])
    ys = [y]
    for t in range(T, T + 3):
        y_t, st = O.ar_recurrent(q, k[:, t:t + 1], v[:, t:t + 1], state=st)
        ys.append(y_t)
    _close(np.concatenate(ys, axis=1), y_all)
    for key in ("m", "d", "u"):
        _close(st[key], st_all[key], 1e-4)


def test_chunked_with_initial_state_equals_concatenation():
    B, T, H, M, D = 1, 24, 2, 16, 16
    q, k, v = seeded(7, B, 2 * T, H, M, D, D, torch.float32)
    _, st = O.ar_chunked(q, k[:, :T], v[:, :T], chunk_size=16, return_state=True)
    y2 = O.ar_chunked(q, k[:, T:], v[:, T:], chunk_size=16, state=st)
    _close(y2, O.brute_ar(q, k, v, scale=0.25)[:, T:])


def test_masked_tokens_output_zero_and_leave_state():
    B, T, H, M, D = 2, 12, 2, 16, 16
    q, k, v = seeded(8, B, T, H, M, D, D, torch.float32)
    mask = np.ones((B, T), np.uint8)
    mask[0, 4] = 0
    mask[1, 0:3] = 0
    y, st = O.ar_recurrent(q, k, v, attention_mask=mask)
    assert np.all(y[0, 4] == 0) and np.all(y[1, 0:3] == 0)
    yb, stb = O.brute_ar_state(q, k, v, attention_mask=mask)
    _close(y, yb)
    _close(st["u"], stb["u"], 1e-4)
    # dropping the masked token entirely gives the same later outputs
    keep = [t for t in range(T) if t != 4]
    y_drop, _ = O.ar_recurrent(q, k[:1, keep], v[:1, keep])
    _close(y[0, 5:], y_drop[0, 4:])
    # the chunked path with a mask agrees with the recurrent one (reference.py:262-282)
    yc = O.ar_chunked(q, k, v, scale=1.0, attention_mask=mask, chunk_size=5)
    _close(yc, y)


def test_closed_form_single_token_and_constant_values():
    q, k, v = seeded(9, 2, 1, 3, 16, 16, 16, torch.float32)
    _close(O.ar_chunked(q, k, v), v.numpy())                 # N = 1: z = v_0 for every latent
    q, k, _ = seeded(10, 1, 40, 2, 16, 16, 8, torch.float32)
    c = torch.randn(1, 1, 2, 8).expand(1, 40, 2, 8).contiguous()
    _close(O.ar_chunked(q, k, c, chunk_size=16), c.numpy())  # constant V -> y = that constant


def test_single_latent_is_causal_softmax_attention():
    """M = 1: alpha = 1 and y_t = softmax_{tau<=t}(q.k_tau) V  (torch SDPA, is_causal)."""
    B, N, H, D = 2, 50, 3, 16
    q, k, v = seeded(11, B, N, H, 1, D, D, torch.float32)
    y = O.ar_chunked(q, k, v, chunk_size=16)
    qq = q[:, 0][None, :, None, :].expand(B, H, N, D)           # same query at every position
    ref = F.scaled_dot_product_attention(qq, k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3), is_causal=True,
                                         scale=D ** -0.5)
    _close(y, ref.permute(0, 2, 1, 3).numpy())


@pytest.mark.parametrize("block,chunk,N", [(16, 16, 48), (32, 16, 64), (64, 32, 128)])
def test_semi_ar_matches_block_sdpa(block, chunk, N):
    B, H, M, D = 2, 3, 5, 16
    q, k, v = seeded(12, B, N, H, M, D, D, torch.float32)
    y, lse_dec, lse_enc = O.semi_ar(q, k, v, block, chunk)
    _close(y, O.brute_semi_ar(q, k, v, block))
    assert lse_dec.shape == (B, H, N) and lse_enc.shape == (B, H, N // block, M)
    # LSE_dec = logsumexp_m of the decoder scores; LSE_enc = logsumexp over tokens < block end
    S = (0.25 * np.einsum("bnhd,hmd->bhnm", k.double().numpy(), q.double().numpy()))
    _close(lse_dec, np.log(np.exp(S).sum(-1)), 1e-5)
    for g in range(N // block):
        _close(lse_enc[:, :, g], np.log(np.exp(S[:, :, : (g + 1) * block]).sum(2)), 1e-5)


def test_semi_ar_full_block_is_noncausal_flare():
    B, N, H, M, D = 1, 32, 2, 8, 16
    q, k, v = seeded(13, B, N, H, M, D, D, torch.float32)
    y, _, _ = O.semi_ar(q, k, v, N, 16)
    z = F.scaled_dot_product_attention(q[None].expand(B, H, M, D), k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3),
                                       scale=0.25)
    ref = F.scaled_dot_product_attention(k.permute(0, 2, 1, 3), q[None].expand(B, H, M, D), z, scale=0.25)
    _close(y, ref.permute(0, 2, 1, 3).numpy())


def test_semi_ar_block_ends_equal_ar():
    """The last token of each block sees exactly the causal prefix: semi-AR == AR there."""
    B, N, H, M, D, blk = 2, 64, 2, 16, 16, 16
    q, k, v = seeded(14, B, N, H, M, D, D, torch.float32)
    ys, _, _ = O.semi_ar(q, k, v, blk, 16)
    ya = O.ar_chunked(q, k, v, chunk_size=16)
    _close(ys[:, blk - 1::blk], ya[:, blk - 1::blk])
    assert np.abs(ys[:, 0] - ya[:, 0]).max() > 1e-3   # and not elsewhere


@pytest.mark.parametrize("block", [1, 4, 16])
def test_semi_state_oracle_without_state_is_block_causal(block):
    """No cached state: the block-causal definition (semi_autoregressive/reference.py:560-597)."""
    B, N, H, M, D = 2, 32, 2, 6, 8
    q, k, v = seeded(30, B, N, H, M, D, D, torch.float32)
    y, _ = O.brute_semi_ar_state(q, k, v, block)
    _close(y, O.brute_semi_ar(q, k, v, block), 1e-12)


def test_semi_state_oracle_continuation_and_final_state():
    """prefill(a + b) == prefill(a) then prefill(b) from its state (split at a block end);
    the state after the tokens is the autoregressive one (independent of the blocking);
    one-token blocks reduce to the autoregressive prefill from the same state."""
    B, N, H, M, D, blk = 2, 48, 2, 5, 8, 8
    q, k, v = seeded(31, B, N, H, M, D, D, torch.float32)
    # a random cached state, as a previous prefill leaves it
    q0, k0, v0 = seeded(32, B, 11, H, M, D, D, torch.float32)
    _, st0 = O.brute_ar_state(q0, k0, v0, scale=0.3)
    y_all, st_all = O.brute_semi_ar_state(q, k, v, blk, state=st0, scale=0.3)
    cut = 3 * blk
    y_a, st_a = O.brute_semi_ar_state(q, k[:, :cut], v[:, :cut], blk, state=st0, scale=0.3)
    y_b, st_b = O.brute_semi_ar_state(q, k[:, cut:], v[:, cut:], blk, state=st_a, scale=0.3)
    _close(np.concatenate([y_a, y_b], axis=1), y_all, 1e-12)
    for key in ("m", "d", "u"):
        _close(st_b[key], st_all[key], 1e-12)
    y_ar, st_ar = O.brute_ar_state(q, k, v, state=st0, scale=0.3)
    for key in ("m", "d", "u"):
        _close(st_all[key], st_ar[key], 1e-10)
    y1, _ = O.brute_semi_ar_state(q, k, v, 1, state=st0, scale=0.3)
    _close(y1, y_ar, 1e-10)
    # closed form: constant values give y = that constant in every block
    vc = torch.full_like(v, 0.75)
    _, stc = O.brute_ar_state(q0, k0, torch.full_like(v0, 0.75), scale=0.3)
    yc, _ = O.brute_semi_ar_state(q, k, vc, blk, state=stc, scale=0.3)
    _close(yc, np.full(yc.shape, 0.75), 1e-12)


def test_golden_fixtures():
    files = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))
    assert files, "no golden fixtures"
    for f in files:
        with np.load(os.path.join(GOLDEN, f), allow_pickle=False) as z:
            kind = str(z["kind"])
            q, k, v = z["q"], z["k"], z["v"]
            if kind == "ar":
                y = O.ar_chunked(q, k, v, scale=float(z["scale"]), chunk_size=int(z["chunk"]))
            elif kind == "semi":
                y, _, _ = O.semi_ar(q, k, v, int(z["block"]), 16, scale=float(z["scale"]))
            else:
                y, _ = O.ar_recurrent(q, k, v, scale=float(z["scale"]))
            _close(y, z["y"], 3e-5)


# --------------------------------------------------------------------------
# Gradient oracle (ar_grads): pinned by the per-token definition (forward
# values) and by central finite differences of that definition.
# --------------------------------------------------------------------------
def _grad_inputs(seed, B, N, H, M, D, Dv, sep_q, sep_k):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(s, generator=g, dtype=torch.float64)
    Q, K, V = r(H, M, D), r(B, N, H, D), r(B, N, H, Dv)
    Qd = r(B, N, H, D) if sep_q else None
    Kd = r(H, M, D) if sep_k else None
    return Q, K, V, Qd, Kd, r(B, N, H, Dv)


@pytest.mark.parametrize("sep_q,sep_k", [(False, False), (True, False), (False, True), (True, True)])
def test_grad_oracle_forward_is_the_definition(sep_q, sep_k):
    Q, K, V, Qd, Kd, _ = _grad_inputs(3, 2, 19, 2, 8, 8, 5, sep_q, sep_k)
    y = O.ar_forward_torch64(Q, K, V, 0.6, Qd, Kd)
    _close(y.numpy(), O.brute_ar(Q, K, V, 0.6, Qd, Kd), 1e-12)


@pytest.mark.parametrize("sep_q,sep_k", [(False, False), (True, False), (False, True), (True, True)])
def test_grad_oracle_matches_finite_differences(sep_q, sep_k):
    """Central differences of sum(brute_ar * dY) (the numpy per-token
    definition, independent of the autograd graph) at every input entry."""
    Q, K, V, Qd, Kd, G = _grad_inputs(5, 1, 6, 1, 4, 3, 2, sep_q, sep_k)
    grads = O.ar_grads(Q, K, V, G, 0.8, Qd, Kd)
    inputs = [Q, K, V, Qd, Kd]
    Gn = G.numpy()
    h = 1e-6
    for idx, (x, gx) in enumerate(zip(inputs, grads)):
        if x is None:
            assert gx is None
            continue
        fd = np.zeros(x.shape)
        for j in range(x.numel()):
            vals = []
            for sgn in (1.0, -1.0):
                xs = [t.clone() if t is not None else None for t in inputs]
                xs[idx].view(-1)[j] += sgn * h
                vals.append(float((O.brute_ar(xs[0], xs[1], xs[2], 0.8, xs[3], xs[4]) * Gn).sum()))
            fd.reshape(-1)[j] = (vals[0] - vals[1]) / (2 * h)
        np.testing.assert_allclose(gx, fd, rtol=1e-6, atol=1e-8)


def test_grad_oracle_single_latent_is_attention_backward():
    """M = 1: alpha = 1 and y is causal softmax attention of the latent's
    scores, whose gradient torch's SDPA backward gives independently."""
    Q, K, V, _, _, G = _grad_inputs(7, 1, 9, 2, 1, 4, 3, False, False)
    dQ, dK, dV, _, _ = O.ar_grads(Q, K, V, G, 0.5)
    q, k, v = (t.clone().requires_grad_(True) for t in (Q, K, V))
    # y_t = sum_{tau<=t} softmax_tau(0.5 k_tau . q) v_tau: attention with query q
    # repeated per token, key k, causal mask -- but the decoder score also
    # depends on k through alpha = softmax over one latent = 1 (no gradient).
    qq = q[:, 0].unsqueeze(0).unsqueeze(2).expand(1, 2, 9, 4)            # [B,H,N,D]
    y = F.scaled_dot_product_attention(qq, k.transpose(1, 2), v.transpose(1, 2), is_causal=True, scale=0.5)
    (y.transpose(1, 2) * G).sum().backward()
    _close(dV, v.grad.numpy(), 1e-10)
    _close(dK, k.grad.numpy(), 1e-10)
    _close(dQ, q.grad.numpy(), 1e-10)


@pytest.mark.parametrize("sep_q,sep_k", [(False, False), (True, True)])
@pytest.mark.parametrize("block", [4, 8])
def test_semi_grad_oracle_forward_is_the_definition(sep_q, sep_k, block):
    Q, K, V, Qd, Kd, _ = _grad_inputs(4, 2, 16, 2, 8, 8, 5, sep_q, sep_k)
    y = O.semi_forward_torch64(Q, K, V, block, 0.6, Qd, Kd)
    _close(y.numpy(), O.brute_semi_ar(Q, K, V, block, 0.6, Qd, Kd), 1e-12)


@pytest.mark.parametrize("sep_q,sep_k", [(False, False), (True, False), (False, True), (True, True)])
def test_semi_grad_oracle_matches_finite_differences(sep_q, sep_k):
    Q, K, V, Qd, Kd, G = _grad_inputs(6, 1, 6, 1, 4, 3, 2, sep_q, sep_k)
    grads = O.semi_grads(Q, K, V, G, 2, 0.8, Qd, Kd)
    inputs = [Q, K, V, Qd, Kd]
    Gn = G.numpy()
    h = 1e-6
    for idx, (x, gx) in enumerate(zip(inputs, grads)):
        if x is None:
            assert gx is None
            continue
        fd = np.zeros(x.shape)
        for j in range(x.numel()):
            vals = []
            for sgn in (1.0, -1.0):
                xs = [t.clone() if t is not None else None for t in inputs]
                xs[idx].view(-1)[j] += sgn * h
                vals.append(float((O.brute_semi_ar(xs[0], xs[1], xs[2], 2, 0.8, xs[3], xs[4]) * Gn).sum()))
            fd.reshape(-1)[j] = (vals[0] - vals[1]) / (2 * h)
        np.testing.assert_allclose(gx, fd, rtol=1e-6, atol=1e-8)


# --------------------------------------------------------------------------
# Stablemax variant (reference autoregressive/stablemax.py, stablemax_triton.py)
# --------------------------------------------------------------------------
def test_stablemax_transform_closed_forms():
    """s(x) = (1+x)^p (x >= 0), (1-x)^-p (x < 0): s(0) = 1, s(1) = 2^p, s(-1) = 2^-p,
    s(3) = 4^p, s(-3) = 4^-p; positive and increasing."""
    for p in (1.0, 2.0, 3.0, 4.0, 2.5):
        s = O.stablemax_transform(np.array([0.0, 1.0, -1.0, 3.0, -3.0]), p)
        np.testing.assert_allclose(s, [1.0, 2.0 ** p, 2.0 ** -p, 4.0 ** p, 4.0 ** -p], rtol=1e-14)
        x = np.linspace(-20, 20, 4001)
        sx = O.stablemax_transform(x, p)
        assert (sx > 0).all() and (np.diff(sx) > 0).all()


@pytest.mark.parametrize("power", [1.0, 2.0, 3.0, 4.0, 2.5])
@pytest.mark.parametrize("chunk", [16, 32, 48])
def test_stablemax_chunked_equals_per_token_definition(power, chunk):
    """The chunked form (stablemax.py:578-635: chunk sums, strict prefixes,
    tril(R W^T) V inside a chunk) equals the per-token definition, ragged N,
    with shared and with separate decoder tensors."""
    rng = np.random.default_rng(11)
    H, M, D, B, N = 2, 24, 16, 2, 77
    q = rng.standard_normal((H, M, D))
    k = rng.standard_normal((B, N, H, D))
    v = rng.standard_normal((B, N, H, D))
    np.testing.assert_allclose(O.stablemax_chunked(q, k, v, power=power, chunk_size=chunk),
                               O.brute_stablemax(q, k, v, power=power), rtol=1e-10, atol=1e-12)
    qd = rng.standard_normal((B, N, H, D))
    kd = rng.standard_normal((H, M, D))
    np.testing.assert_allclose(
        O.stablemax_chunked(q, k, v, power=power, chunk_size=chunk, Q_dec=qd, K_dec=kd, scale=0.3),
        O.brute_stablemax(q, k, v, power=power, Q_dec=qd, K_dec=kd, scale=0.3), rtol=1e-10, atol=1e-12)


def test_stablemax_zero_scores_give_the_causal_mean():
    """Q = 0: every score is 0, s = 1 for every (token, latent), so z_t is the mean of
    v over tau <= t for every latent and y_t (a convex combination of the z) is that
    mean, whatever the power and the decoder."""
    rng = np.random.default_rng(12)
    H, M, D, B, N = 2, 8, 4, 1, 30
    q = np.zeros((H, M, D))
    k = rng.standard_normal((B, N, H, D))
    v = rng.standard_normal((B, N, H, D))
    mean = np.cumsum(v, axis=1) / np.arange(1, N + 1)[None, :, None, None]
    for p in (1.0, 3.0):
        np.testing.assert_allclose(O.brute_stablemax(q, k, v, power=p), mean, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(O.stablemax_chunked(q, k, v, power=p, chunk_size=16), mean, rtol=1e-12, atol=1e-12)


def test_stablemax_first_token_is_its_value():
    """N = 1: z_0 = v_0 for every latent, so y_0 = v_0."""
    rng = np.random.default_rng(13)
    q = rng.standard_normal((3, 16, 8))
    k = rng.standard_normal((2, 1, 3, 8))
    v = rng.standard_normal((2, 1, 3, 8))
    np.testing.assert_allclose(O.brute_stablemax(q, k, v, power=2.0), v, rtol=1e-13)


def test_chunk_summaries_merge_to_the_whole_sequence_state():
    """Phase 1's per-chunk (max, den, num), merged over all chunks with the
    inf-safe online-softmax merge (reference.py:160-187), equal the state
    {m, d, u} of the whole sequence from the per-token definition
    (brute_ar_state); with chunk = N they are that state directly."""
    rng = np.random.default_rng(21)
    H, M, D, B, N = 2, 16, 8, 2, 70
    q = rng.standard_normal((H, M, D)) * 0.7
    k = rng.standard_normal((B, N, H, D))
    v = rng.standard_normal((B, N, H, D))
    _, st = O.brute_ar_state(q, k, v, scale=D ** -0.5)
    for chunk in (16, 24, 70):
        mx, den, num = O.chunk_summaries(q, k, v, chunk, scale=D ** -0.5)
        m, d, u = mx[:, 0], den[:, 0], num[:, 0]
        for c in range(1, mx.shape[1]):
            mn = np.maximum(m, mx[:, c])
            a, b = np.exp(m - mn), np.exp(mx[:, c] - mn)
            d, u, m = d * a + den[:, c] * b, u * a[..., None] + num[:, c] * b[..., None], mn
        np.testing.assert_allclose(m.reshape(B, H, M), st["m"], rtol=1e-12)
        np.testing.assert_allclose(d.reshape(B, H, M), st["d"], rtol=1e-10)
        np.testing.assert_allclose(u.reshape(B, H, M, D), st["u"], rtol=1e-9, atol=1e-12)


# --------------------------------------------------------------------------
# Stablemax gradient oracle (stablemax_grads): pinned by the per-token
# definition (forward values, powers 1-4 and 2.5) and central finite
# differences of brute_stablemax.
# --------------------------------------------------------------------------
@pytest.mark.parametrize("power", [1.0, 2.0, 2.5, 4.0])
@pytest.mark.parametrize("sep_q,sep_k", [(False, False), (True, True)])
def test_stablemax_grad_oracle_forward_is_the_definition(power, sep_q, sep_k):
    Q, K, V, Qd, Kd, _ = _grad_inputs(13, 2, 17, 2, 8, 8, 5, sep_q, sep_k)
    y = O.stablemax_forward_torch64(Q, K, V, power, 0.7, Qd, Kd)
    _close(y.numpy(), O.brute_stablemax(Q, K, V, power, 0.7, Qd, Kd), 1e-12)


@pytest.mark.parametrize("power", [2.0, 2.5])
@pytest.mark.parametrize("sep_q,sep_k", [(False, False), (True, False), (False, True), (True, True)])
def test_stablemax_grad_oracle_matches_finite_differences(power, sep_q, sep_k):
    """Central differences of sum(brute_stablemax * dY) at every input entry (the
    scores cross 0, where the transform's two branches meet with equal value and
    slope p)."""
    Q, K, V, Qd, Kd, G = _grad_inputs(17, 1, 6, 1, 4, 3, 2, sep_q, sep_k)
    grads = O.stablemax_grads(Q, K, V, G, power, 0.8, Qd, Kd)
    inputs = [Q, K, V, Qd, Kd]
    Gn = G.numpy()
    h = 1e-6
    for idx, (x, gx) in enumerate(zip(inputs, grads)):
        if x is None:
            assert gx is None
            continue
        fd = np.zeros(x.shape)
        for j in range(x.numel()):
            vals = []
            for sgn in (1.0, -1.0):
                xs = [t.clone() if t is not None else None for t in inputs]
                xs[idx].view(-1)[j] += sgn * h
                vals.append(float((O.brute_stablemax(xs[0], xs[1], xs[2], power, 0.8, xs[3], xs[4]) * Gn).sum()))
            fd.reshape(-1)[j] = (vals[0] - vals[1]) / (2 * h)
        np.testing.assert_allclose(gx, fd, rtol=1e-6, atol=1e-8)
