"""GPU parity of the backward (flare_ar_backward through AutoRegressiveFLARE)
against the fp64 autograd oracle (oracle/flare_oracle.py: ar_grads).

Mirrors testing/autoregressive/test_flare.py:370-427 (decoder-flag backward
against the torch reference) and widens it to multi-chunk, ragged, bf16 and
sharp-score cases.

Tolerances:
  * the reference's own backward bar for fp32 inputs at its test shape,
    torch.testing.assert_close(rtol=1e-2, atol=1e-3) (test_flare.py:421-427);
  * elsewhere a scale-free bar: max |g - g_ref| <= tol * max(max |g_ref|, 1e-2)
    per gradient tensor (the floor covers gradients that vanish exactly, such
    as dQ and dK for a one-token sequence, where y_0 = v_0); tol = 1e-4 for
    fp32 inputs (fp32 accumulation over up to a few thousand tokens) and 2e-2
    for bf16 inputs (bf16 inputs and bf16 gradients, each rounded at 2^-8
    relative).
"""
import math
import sys

import numpy as np
import pytest
import torch

import flare_oracle as O
from _util import to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(*args):
    print("CASE", *args, flush=True)
    sys.stdout.flush()


def _inputs(seed, B, N, H, M, D, Dv, dtype, sep_q, sep_k, q_std=1.0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(s, generator=g)
    Q = r(H, M, D) * q_std
    K, V = r(B, N, H, D), r(B, N, H, Dv)
    Qd = r(B, N, H, D) if sep_q else None
    Kd = r(H, M, D) * q_std if sep_k else None
    G = r(B, N, H, Dv)
    cast = lambda t: None if t is None else t.to(dtype)
    return tuple(cast(t) for t in (Q, K, V, Qd, Kd, G))


def _run(Q, K, V, Qd, Kd, G, scale, chunk=None):
    from causal_flare import flare_autoregressive_triton
    leaves = [None if t is None else t.to(DEV).requires_grad_(True) for t in (Q, K, V, Qd, Kd)]
    y = flare_autoregressive_triton(leaves[0], leaves[1], leaves[2], scale=scale, chunk_size=chunk,
                                    Q_dec=leaves[3], K_dec=leaves[4])
    (y.float() * G.to(DEV).float()).sum().backward()
    return y, [None if t is None else t.grad for t in leaves]


def _check(grads, ref, tol, what):
    for name, g, r in zip(("dQ", "dK", "dV", "dQ_dec", "dK_dec"), grads, ref):
        if r is None:
            assert g is None, f"{what}: unexpected {name}"
            continue
        a = to_np(g).astype(np.float64)
        assert a.shape == r.shape, (what, name, a.shape, r.shape)
        assert np.isfinite(a).all(), f"{what}: non-finite {name}"
        err = np.abs(a - r).max() / max(np.abs(r).max(), 1e-2)
        print(f"  {what}: {name} normalised max error {err:.3e}")
        assert err <= tol, f"{what}: {name} normalised max error {err:.3e} > {tol}"


@pytest.mark.parametrize("d_score,d_value", [(16, 16), (64, 128)])
def test_decoder_flags_backward_reference_shape(d_score, d_value):
    """test_flare.py:370-427 at its shape and tolerance."""
    B, N, H, M = 1, 16, 2, 16
    scale = 1.0 / math.sqrt(d_score)
    for sep_q in (False, True):
        for sep_k in (False, True):
            _case("bwd_ref_shape", d_score, d_value, sep_q, sep_k)
            Q, K, V, Qd, Kd, G = _inputs(2029, B, N, H, M, d_score, d_value, torch.float32, sep_q, sep_k)
            y, grads = _run(Q, K, V, Qd, Kd, G, scale, chunk=16)
            ref = O.ar_grads(Q, K, V, G, scale, Qd, Kd)
            for name, g, r in zip(("q", "k", "v", "q_dec", "k_dec"), grads, ref):
                if r is None:
                    continue
                torch.testing.assert_close(g.cpu().double(), torch.as_tensor(r), rtol=1e-2, atol=1e-3,
                                           msg=lambda m: f"{name} sep_q={sep_q} sep_k={sep_k}: {m}")


@pytest.mark.parametrize("q_dec_mode", ["none", "k_enc", "rand"])
@pytest.mark.parametrize("k_dec_mode", ["none", "q_enc", "rand"])
def test_backward_aliasing_modes_fp32(q_dec_mode, k_dec_mode):
    """The 3x3 decoder aliasing modes (test_flare.py:430-490): a decoder tensor
    that is the encoder tensor itself gets its gradient folded into dK / dQ."""
    from causal_flare import flare_autoregressive_triton
    _case("bwd_alias", q_dec_mode, k_dec_mode)
    B, N, H, M, D, Dv = 2, 150, 2, 32, 32, 48
    Q, K, V, Qd, Kd, G = _inputs(11, B, N, H, M, D, Dv, torch.float32, True, True)
    q, k, v = (t.to(DEV).requires_grad_(True) for t in (Q, K, V))
    qd = {"none": None, "k_enc": k, "rand": Qd.to(DEV).requires_grad_(True)}[q_dec_mode]
    kd = {"none": None, "q_enc": q, "rand": Kd.to(DEV).requires_grad_(True)}[k_dec_mode]
    y = flare_autoregressive_triton(q, k, v, scale=0.2, Q_dec=qd, K_dec=kd)
    (y * G.to(DEV)).sum().backward()
    ref = O.ar_grads(Q, K, V, G, 0.2, Qd if q_dec_mode == "rand" else None, Kd if k_dec_mode == "rand" else None)
    got = [q.grad, k.grad, v.grad, qd.grad if q_dec_mode == "rand" else None,
           kd.grad if k_dec_mode == "rand" else None]
    _check(got, ref, 1e-4, f"alias q_dec={q_dec_mode} k_dec={k_dec_mode}")


@pytest.mark.parametrize("B,N,H,M,D,Dv", [(1, 1, 1, 16, 16, 16), (2, 63, 1, 16, 32, 16), (1, 65, 2, 48, 16, 80),
                                          (2, 300, 2, 64, 64, 64), (1, 2100, 1, 32, 32, 32)])
@pytest.mark.parametrize("sep", [(False, False), (True, True)])
def test_backward_shapes_fp32(B, N, H, M, D, Dv, sep):
    """Ragged final chunks, one-token sequences, many chunks (the reverse carry)."""
    _case("bwd_fp32", B, N, H, M, D, Dv, sep)
    Q, K, V, Qd, Kd, G = _inputs(5, B, N, H, M, D, Dv, torch.float32, *sep)
    scale = 1.0 / math.sqrt(D)
    _, grads = _run(Q, K, V, Qd, Kd, G, scale)
    _check(grads, O.ar_grads(Q, K, V, G, scale, Qd, Kd), 1e-4, f"fp32 {B, N, H, M, D, Dv, sep}")


@pytest.mark.parametrize("q_std", [2.0, 4.0])
def test_backward_sharp_scores_fp32(q_std):
    """Large scores: running maxima move by tens within a chunk, so the factors
    e^{s - L} span many orders of magnitude."""
    _case("bwd_sharp", q_std)
    Q, K, V, Qd, Kd, G = _inputs(8, 1, 400, 2, 32, 32, 32, torch.float32, False, False, q_std=q_std)
    _, grads = _run(Q, K, V, Qd, Kd, G, 1.0)
    _check(grads, O.ar_grads(Q, K, V, G, 1.0, Qd, Kd), 1e-4, f"sharp q_std={q_std}")


@pytest.mark.parametrize("M,D,N", [(128, 64, 1000), (256, 128, 300), (64, 64, 1100), (64, 128, 77)])
@pytest.mark.parametrize("sep", [(False, False), (True, False), (False, True), (True, True)])
def test_backward_bf16(M, D, N, sep):
    """bf16 inputs: dK / dQ_dec and dQ / dK_dec run as bf16 MFMA contractions (hi/lo
    split gradients) for these shapes, in all four decoder-weight modes; N = 1100
    leaves a ragged last token group of the dQ partial sums."""
    _case("bwd_bf16", M, D, N, sep)
    Q, K, V, Qd, Kd, G = _inputs(9, 1, N, 2, M, D, D, torch.bfloat16, *sep)
    Q = (Q.float() / math.sqrt(D)).to(torch.bfloat16)
    if Kd is not None:   # latent decoder keys scaled like the latent queries
        Kd = (Kd.float() / math.sqrt(D)).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    y, grads = _run(Q, K, V, Qd, Kd, G, scale)
    assert y.dtype == torch.bfloat16 and all(g is None or g.dtype == torch.bfloat16 for g in grads)
    # the reference's bf16 bar: 2e-2, 3e-2 for D >= 128 (test_block_causal.py:178-255)
    tol = 3e-2 if D >= 128 else 2e-2
    _check(grads, O.ar_grads(Q, K, V, G, scale, Qd, Kd), tol, f"bf16 M={M} D={D} N={N} sep={sep}")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
def test_backward_bf16_score_jump(M, D):
    """A token whose scores pass the chunk's starting log-den by far more than 2^64
    (one K row scaled by 300): the pair sums of that chunk take the exact per-pair
    path instead of the factorised MFMA form."""
    _case("bwd_bf16_jump", M, D)
    N = 200
    Q, K, V, Qd, Kd, G = _inputs(21, 1, N, 2, M, D, D, torch.bfloat16, False, False)
    Q = (Q.float() / math.sqrt(D)).to(torch.bfloat16)
    K = K.float()
    K[:, 45] *= 300.0
    K = K.to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    y, grads = _run(Q, K, V, Qd, Kd, G, scale)
    tol = 3e-2 if D >= 128 else 2e-2
    _check(grads, O.ar_grads(Q, K, V, G, scale, Qd, Kd), tol, f"bf16 jump M={M} D={D}")


@pytest.mark.parametrize("M,D,N,jumps", [(128, 64, 2500, ()), (256, 128, 1500, ()), (128, 64, 1500, (650, 700)),
                                         (256, 128, 1100, (1000,))])
def test_backward_bf16_long_walk(M, D, N, jumps, monkeypatch):
    """The chunk starting states walked over long chunks (1024 tokens: 16 tiles each, as
    config 3's 4096-token chunks hold 64): the running state written at every 32-token
    chunk across tiles, with K rows scaled by 12 (scores up to about 8, past the lazy
    references of many latents) that move a reference in the first (token 650 of its
    tile's 640 .. 703) and the second half (700, 1000) of a tile.  (Rows scaled by 40 put
    some gradients past the bf16 bar on every path, the fp32 kernels included: da = alpha
    (gz - g . y) cancels where alpha peaks, against the saved bf16 y.)"""
    _case("bwd_bf16_long_walk", M, D, N, jumps)
    monkeypatch.setenv("FLARE_BWD_WALK_CHUNK", "1024")
    Q, K, V, Qd, Kd, G = _inputs(23, 1, N, 2, M, D, D, torch.bfloat16, False, False)
    Q = (Q.float() / math.sqrt(D)).to(torch.bfloat16)
    if jumps:
        K = K.float()
        for t in jumps:
            K[:, t] *= 12.0
        K = K.to(torch.bfloat16)
    scale = 1.0 / math.sqrt(D)
    y, grads = _run(Q, K, V, Qd, Kd, G, scale)
    tol = 3e-2 if D >= 128 else 2e-2
    _check(grads, O.ar_grads(Q, K, V, G, scale, Qd, Kd), tol, f"bf16 long walk M={M} D={D} N={N} jumps={jumps}")


@pytest.mark.parametrize("M,D,N", [(128, 64, 300), (256, 128, 200)])
@pytest.mark.parametrize("sep", [(False, False), (True, True)])
def test_backward_fp16(M, D, N, sep):
    """fp16 inputs (computed in fp16 by the reference, training.py:315-326), bar of
    _get_allclose_tols for 16-bit inputs with the D >= 128 allowance."""
    _case("bwd_fp16", M, D, N, sep)
    Q, K, V, Qd, Kd, G = _inputs(19, 1, N, 2, M, D, D, torch.float16, *sep)
    Q = (Q.float() / math.sqrt(D)).to(torch.float16)
    if Kd is not None:
        Kd = (Kd.float() / math.sqrt(D)).to(torch.float16)
    scale = 1.0 / math.sqrt(D)
    y, grads = _run(Q, K, V, Qd, Kd, G, scale)
    assert y.dtype == torch.float16 and all(g is None or g.dtype == torch.float16 for g in grads)
    tol = 3e-2 if D >= 128 else 2e-2
    _check(grads, O.ar_grads(Q, K, V, G, scale, Qd, Kd), tol, f"fp16 M={M} D={D} N={N} sep={sep}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,D,Dv,N", [(48, 32, 96, 200), (64, 64, 256, 150), (32, 64, 32, 100),
                                      (128, 64, 192, 130)])
def test_backward_16bit_other_value_widths(dtype, M, D, Dv, N):
    """16-bit inputs away from the square 64 / 128 heads: the chunk summary on its
    scalar kernel (M or Dv outside the MFMA instances), GV on the MFMA at Dv = 32 and
    96, and bwd_dv with eight 64-column value slabs (Dv > 128)."""
    _case("bwd_16bit_widths", str(dtype), M, D, Dv, N)
    Q, K, V, Qd, Kd, G = _inputs(23, 1, N, 2, M, D, Dv, dtype, False, False)
    Q = (Q.float() / math.sqrt(D)).to(dtype)
    scale = 1.0 / math.sqrt(D)
    y, grads = _run(Q, K, V, Qd, Kd, G, scale)
    assert y.dtype == dtype and all(g is None or g.dtype == dtype for g in grads)
    tol = 3e-2 if max(D, Dv) >= 128 else 2e-2
    _check(grads, O.ar_grads(Q, K, V, G, scale, Qd, Kd), tol, f"{dtype} M={M} D={D} Dv={Dv} N={N}")


def test_backward_c_abi_rejects_bad_arguments():
    from causal_flare import _lib
    lib = _lib.lib()
    B, N, H, M, D = 1, 16, 1, 16, 16
    t = torch.zeros(64, device=DEV)
    P = _lib.ptr
    need = lib.flare_ar_backward_workspace_size(B, N, H, M, D, D)
    rc = lib.flare_ar_backward(P(t), P(t), P(t), None, None, 0, B, N, H, M, D, D, 1.0, P(t), P(t), P(t), P(t),
                               P(t), None, None, P(t), need - 1, None)
    assert rc != 0 and b"workspace" in lib.flare_last_error()
    rc = lib.flare_ar_backward(P(t), P(t), P(t), None, None, 0, B, N, H, 512, D, D, 1.0, P(t), P(t), P(t), P(t),
                               P(t), None, None, P(t), need, None)
    assert rc != 0 and b"M=512" in lib.flare_last_error()


# --------------------------------------------------------------------------
# flare_recurrent_triton (served by the chunked kernels; Y [B, H, T, D])
# --------------------------------------------------------------------------
@pytest.mark.parametrize("block_t", [1, 16])
def test_recurrent_decoder_variants_backward_reference_shape(block_t):
    """test_flare.py:222-281: 3x3 decoder modes, forward at rtol 1e-4 / atol 1e-5,
    gradients at rtol 1e-2 / atol 1e-3, against the fp64 definition."""
    from causal_flare import flare_recurrent_triton
    B, N, H, M, D = 1, 16, 2, 16, 16
    scale = 1.0 / math.sqrt(D)
    g = torch.Generator().manual_seed(321)
    r = lambda *s: torch.randn(s, generator=g)
    Q, K, V, Qd, Kd = r(H, M, D), r(B, N, H, D), r(B, N, H, D), r(B, N, H, D), r(H, M, D)
    G = r(B, H, N, D)
    for qm in ("none", "k_enc", "rand"):
        for km in ("none", "q_enc", "rand"):
            _case("recurrent_ref_shape", block_t, qm, km)
            q, k, v = (t.to(DEV).requires_grad_(True) for t in (Q, K, V))
            qd = {"none": None, "k_enc": k, "rand": Qd.to(DEV).requires_grad_(True)}[qm]
            kd = {"none": None, "q_enc": q, "rand": Kd.to(DEV).requires_grad_(True)}[km]
            y = flare_recurrent_triton(q, k, v, scale=scale, Q_dec=qd, K_dec=kd, block_t=block_t)
            assert y.shape == (B, H, N, D) and y.dtype == torch.float32
            (y * G.to(DEV)).sum().backward()
            qd_o = Qd if qm == "rand" else None
            kd_o = Kd if km == "rand" else None
            y_ref = O.brute_ar(Q, K, V, scale, qd_o, kd_o).transpose(0, 2, 1, 3)
            torch.testing.assert_close(y.detach().cpu().double(), torch.as_tensor(y_ref), rtol=1e-4, atol=1e-5)
            ref = O.ar_grads(Q, K, V, G.permute(0, 2, 1, 3), scale, qd_o, kd_o)
            got = [q.grad, k.grad, v.grad, qd.grad if qm == "rand" else None, kd.grad if km == "rand" else None]
            for name, a, b in zip(("q", "k", "v", "q_dec", "k_dec"), got, ref):
                if b is None:
                    continue
                torch.testing.assert_close(a.cpu().double(), torch.as_tensor(b), rtol=1e-2, atol=1e-3,
                                           msg=lambda m: f"recurrent {name} q_dec={qm} k_dec={km}: {m}")


def test_recurrent_bf16_matches_chunked():
    """bf16, MFMA shapes: the recurrent entry point equals the chunked one in [B, H, T, D]."""
    from causal_flare import flare_autoregressive_triton, flare_recurrent_triton
    _case("recurrent_bf16")
    B, N, H, M, D = 2, 700, 2, 128, 64
    q, k, v, _, _, _ = _inputs(17, B, N, H, M, D, D, torch.bfloat16, False, False, q_std=D ** -0.5)
    y = flare_recurrent_triton(q.to(DEV), k.to(DEV), v.to(DEV))
    y2 = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV))
    assert y.dtype == torch.bfloat16 and y.shape == (B, H, N, D)
    assert torch.equal(y, y2.permute(0, 2, 1, 3))


# --------------------------------------------------------------------------
# Block-causal (semi-autoregressive) backward
# --------------------------------------------------------------------------
def _run_semi(Q, K, V, Qd, Kd, G, block, scale):
    from causal_flare import flare_semi_autoregressive_trition
    leaves = [None if t is None else t.to(DEV).requires_grad_(True) for t in (Q, K, V, Qd, Kd)]
    y, aux = flare_semi_autoregressive_trition(leaves[0], leaves[1], leaves[2], block_size=block,
                                               chunk_size=min(block, 64), scale=scale, Q_dec=leaves[3],
                                               K_dec=leaves[4])
    (y.float() * G.to(DEV).float()).sum().backward()
    return y, [None if t is None else t.grad for t in leaves]


@pytest.mark.parametrize("sep", [(False, False), (True, True)])
def test_semi_backward_reference_shape_bf16(sep):
    """test_block_causal.py:433-530: B=1, N=64, H=2, M=16, D=16, block 32, bf16,
    rtol = atol = 2e-2."""
    _case("semi_bwd_ref_shape", sep)
    Q, K, V, Qd, Kd, G = _inputs(6, 1, 64, 2, 16, 16, 16, torch.bfloat16, *sep)
    scale = 16 ** -0.5
    _, grads = _run_semi(Q, K, V, Qd, Kd, G, 32, scale)
    ref = O.semi_grads(Q, K, V, G, 32, scale, Qd, Kd)
    for name, g, r in zip(("q", "k", "v", "q_dec", "k_dec"), grads, ref):
        if r is None:
            continue
        torch.testing.assert_close(g.cpu().double(), torch.as_tensor(r), rtol=2e-2, atol=2e-2,
                                   msg=lambda m: f"semi {name}: {m}")


def test_semi_backward_fp16():
    """Block-causal backward with fp16 inputs, the reference's 16-bit bar."""
    _case("semi_bwd_fp16")
    Q, K, V, Qd, Kd, G = _inputs(8, 1, 256, 2, 128, 64, 64, torch.float16, False, False)
    Q = (Q.float() / 8.0).to(torch.float16)
    scale = 64 ** -0.5
    _, grads = _run_semi(Q, K, V, Qd, Kd, G, 64, scale)
    ref = O.semi_grads(Q, K, V, G, 64, scale, Qd, Kd)
    _check(grads, ref, 2e-2, "semi fp16")


@pytest.mark.parametrize("block", [16, 64])
@pytest.mark.parametrize("sep", [(False, False), (True, False), (False, True)])
def test_semi_backward_fp32(block, sep):
    _case("semi_bwd_fp32", block, sep)
    Q, K, V, Qd, Kd, G = _inputs(12, 2, 256, 2, 32, 32, 48, torch.float32, *sep)
    scale = 32 ** -0.5
    _, grads = _run_semi(Q, K, V, Qd, Kd, G, block, scale)
    _check(grads, O.semi_grads(Q, K, V, G, block, scale, Qd, Kd), 1e-4, f"semi fp32 block={block} sep={sep}")


def test_semi_backward_large_bf16():
    """test_block_causal.py:536-580 (B=4, M=64, D=32, block 256; N halved to keep the
    fp64 oracle small), rtol = atol = 3e-2, and the scale-free bar."""
    _case("semi_bwd_large")
    Q, K, V, Qd, Kd, G = _inputs(8, 4, 4096, 2, 64, 32, 32, torch.bfloat16, False, False)
    scale = 32 ** -0.5
    _, grads = _run_semi(Q, K, V, Qd, Kd, G, 256, scale)
    ref = O.semi_grads(Q, K, V, G, 256, scale)
    for name, g, r in zip(("q", "k", "v"), grads, ref):
        torch.testing.assert_close(g.cpu().double(), torch.as_tensor(r), rtol=3e-2, atol=3e-2,
                                   msg=lambda m: f"semi large {name}: {m}")
    _check(grads, ref, 2e-2, "semi large bf16")
