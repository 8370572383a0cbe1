"""CPU oracle for the causal FLARE forward paths -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker or as the timed CPU baseline.
The product package never imports it; there is no CPU fallback in the product.

Two layers:

* ``ar_chunked`` / ``ar_recurrent`` / ``semi_ar`` call the fp32 C restatement in
  ``flare_oracle.c`` (built by ``oracle/Makefile`` into ``oracle/_build``).
  They follow, in order:
    - ``causal_flare/autoregressive/reference.py:203-512`` (chunked forward)
    - ``causal_flare/autoregressive/inference.py:231-351`` (prefill / decode)
    - ``causal_flare/semi_autoregressive/reference.py:308-536`` (block-causal)
* ``brute_*`` are fp64 numpy restatements of the definitions the reference
  uses as its own ground truth:
    - ``brute_ar``: the per-token two-SDPA oracle, ``reference.py:15-47``
    - ``brute_semi_ar``: the per-block two-SDPA oracle, ``semi_autoregressive/reference.py:560-597``
    - ``brute_ar_state``: the same definition continued from a cached state
      ``{m, d, u}`` (``inference.py:66-120``), with an optional token mask.
    - ``brute_semi_ar_state``: the block-causal definition continued from a
      cached state (the semi-AR cached prefill / block decode, which the
      reference leaves as stubs).
    - ``chunk_summaries``: phase 1's per-chunk (max, den, num), fp64.
    - ``stablemax_grads``: fp64 autograd of that definition (the stablemax backward's
      ground truth), pinned by finite differences of ``brute_stablemax``;
    - ``brute_stablemax``: the stablemax variant's per-token definition
      (``autoregressive/stablemax_triton.py:1718-1731``), and
      ``stablemax_chunked``, its chunked form (``stablemax.py:578-635``).
  They are the pins for the C restatement (see tests/test_oracle.py).
* ``ar_grads``: fp64 torch autograd of ``ar_forward_torch64`` (the same
  definition with cumulative sums), the ground truth of the backward; pinned
  by ``brute_ar`` (forward values) and by central finite differences;
  ``semi_grads`` likewise for the block-causal forward (pinned by
  ``brute_semi_ar`` and finite differences).

Parity status: every C entry point is pinned by fp64 brute force, by
invariants (chunk-size independence, prefill/decode continuation, state
continuation, semi-AR/AR agreement at block ends) and by closed forms
(N=1, constant V, M=1 via torch SDPA).  No function here is "parity unpinned".
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libflare_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build(force: bool = False) -> str:
    """Compile the C oracle with its Makefile (gcc, OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "_build/libflare_oracle.so"],
                       check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        i = ctypes.c_int
        f = ctypes.c_float
        lib.oracle_ar_chunked.argtypes = [_f32p] * 5 + [_u8p] + [_f32p] * 3 + [i] * 6 + [f, i, i] + [_f32p] * 4 + [i]
        lib.oracle_ar_recurrent.argtypes = [_f32p] * 5 + [_u8p] + [_f32p] * 3 + [i] * 6 + [f, i] + [_f32p] * 4 + [i]
        lib.oracle_semi_ar.argtypes = [_f32p] * 5 + [i] * 6 + [f, i, i] + [_f32p] * 3 + [i]
        for fn in (lib.oracle_ar_chunked, lib.oracle_ar_recurrent, lib.oracle_semi_ar):
            fn.restype = ctypes.c_int
        _lib = lib
    return _lib


def _f32(x):
    if x is None:
        return None
    if hasattr(x, "detach"):  # torch tensor
        x = x.detach().float().cpu().numpy()
    return np.ascontiguousarray(x, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_f32p)


def _u8(mask):
    if mask is None:
        return None, None
    if hasattr(mask, "detach"):
        mask = mask.detach().cpu().numpy()
    m = np.ascontiguousarray(mask != 0, dtype=np.uint8)
    return m, m.ctypes.data_as(_u8p)


def resolve_scale(scale, head_dim: int) -> float:
    """``_common.py:201-204``: 1.0 when D <= 8, else D**-0.5."""
    if scale is not None:
        return float(scale)
    return 1.0 if head_dim <= 8 else head_dim ** -0.5


def resolve_reference_chunk_size(N: int, M: int, D_score: int, chunk_size=None) -> int:
    """``reference.py:190-200`` (the PyTorch path's own chunk policy)."""
    if chunk_size is not None:
        return int(chunk_size)
    if D_score <= 32 and M <= 64 and N >= 1024:
        return 64
    if D_score <= 64 and M <= 128 and N >= 1024:
        return 128
    return max(64, min(2048, max(1, N // 2)))


def _shared(Q_dec, K_dec):
    return Q_dec is None and K_dec is None


def _state_arrays(state):
    if state is None:
        return None, None, None
    return _f32(state["m"]), _f32(state["d"]), _f32(state["u"])


def ar_chunked(Q, K, V, scale=None, chunk_size=None, Q_dec=None, K_dec=None, state=None,
               attention_mask=None, return_state=False, nthreads=0):
    """fp32 chunked causal FLARE forward (reference.py:203-512). Returns fp32 numpy."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    Qd, Kd = _f32(Q_dec), _f32(K_dec)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    C = resolve_reference_chunk_size(N, M, Dk, chunk_size)
    mask, maskp = _u8(attention_mask)
    m0, d0, u0 = _state_arrays(state)
    Y = np.zeros((B, N, H, Dv), np.float32)
    mo = np.empty((B, H, M), np.float32)
    do = np.empty((B, H, M), np.float32)
    uo = np.empty((B, H, M, Dv), np.float32)
    rc = _load().oracle_ar_chunked(_ptr(Q), _ptr(K), _ptr(V), _ptr(Qd), _ptr(Kd), maskp,
                                   _ptr(m0), _ptr(d0), _ptr(u0), B, N, H, M, Dk, Dv, scale, C,
                                   int(_shared(Q_dec, K_dec)), _ptr(Y), _ptr(mo), _ptr(do), _ptr(uo),
                                   int(nthreads))
    assert rc == 0, rc
    if return_state:
        return Y, {"m": mo, "d": do, "u": uo}
    return Y


def ar_recurrent(Q, K, V, state=None, scale=1.0, attention_mask=None, Q_dec=None, K_dec=None,
                 nthreads=0):
    """fp32 tokenwise prefill (inference.py:231-315); decode is T=1 (:318-351)."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    Qd, Kd = _f32(Q_dec), _f32(K_dec)
    H, M, Dk = Q.shape
    B, T, _, Dv = V.shape
    mask, maskp = _u8(attention_mask)
    m0, d0, u0 = _state_arrays(state)
    Y = np.zeros((B, T, H, Dv), np.float32)
    mo = np.empty((B, H, M), np.float32)
    do = np.empty((B, H, M), np.float32)
    uo = np.empty((B, H, M, Dv), np.float32)
    rc = _load().oracle_ar_recurrent(_ptr(Q), _ptr(K), _ptr(V), _ptr(Qd), _ptr(Kd), maskp,
                                     _ptr(m0), _ptr(d0), _ptr(u0), B, T, H, M, Dk, Dv,
                                     float(scale), int(_shared(Q_dec, K_dec)), _ptr(Y), _ptr(mo),
                                     _ptr(do), _ptr(uo), int(nthreads))
    assert rc == 0, rc
    return Y, {"m": mo, "d": do, "u": uo}


def semi_ar(Q, K, V, block_size, chunk_size, scale=None, Q_dec=None, K_dec=None, nthreads=0):
    """fp32 block-causal forward (semi reference.py:308-536). Returns (Y, LSE_dec, LSE_enc)."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    Qd, Kd = _f32(Q_dec), _f32(K_dec)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    NB = N // block_size
    Y = np.zeros((B, N, H, Dv), np.float32)
    lse_dec = np.empty((B, H, N), np.float32)
    lse_enc = np.empty((B, H, NB, M), np.float32)
    rc = _load().oracle_semi_ar(_ptr(Q), _ptr(K), _ptr(V), _ptr(Qd), _ptr(Kd), B, N, H, M, Dk, Dv,
                                scale, int(block_size), int(chunk_size), _ptr(Y), _ptr(lse_dec),
                                _ptr(lse_enc), int(nthreads))
    assert rc == 0, rc
    return Y, lse_dec, lse_enc


# --------------------------------------------------------------------------
# fp64 brute-force definitions (the pins)
# --------------------------------------------------------------------------

def _f64(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach().double().cpu().numpy()
    return np.asarray(x, dtype=np.float64)


def _softmax(x, axis=-1):
    x = x - x.max(axis=axis, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=axis, keepdims=True)


def brute_ar(Q, K, V, scale=None, Q_dec=None, K_dec=None):
    """reference.py:15-47: z_t = SDPA(Q, K[:t+1], V[:t+1]); y_t = SDPA(Qdec_t, Kdec, z_t). fp64."""
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    Qd = _f64(Q_dec) if Q_dec is not None else K
    Kd = _f64(K_dec) if K_dec is not None else Q
    S = scale * np.einsum("bnhd,hmd->bhnm", K, Q)             # encoder scores
    A = scale * np.einsum("bnhd,hmd->bhnm", Qd, Kd)           # decoder scores
    Vt = V.transpose(0, 2, 1, 3)                               # [B,H,N,Dv]
    Y = np.empty((B, H, N, Dv))
    for t in range(N):
        P = _softmax(S[:, :, : t + 1, :], axis=2)              # over tau <= t
        Z = np.einsum("bhtm,bhtd->bhmd", P, Vt[:, :, : t + 1])
        alpha = _softmax(A[:, :, t, :], axis=-1)
        Y[:, :, t] = np.einsum("bhm,bhmd->bhd", alpha, Z)
    return Y.transpose(0, 2, 1, 3)


def chunk_summaries(Q, K, V, chunk, scale=None):
    """Per-chunk encoder summaries of the chunked forward's phase 1
    (flare_chunk_prepare, training.py:914-1018; reference.py:240-300): for chunk c
    and latent m, max_c = max over the chunk's tokens of s = scale k . q_m (natural
    log units), den_c = sum exp(s - max_c), num_c = sum exp(s - max_c) v.  fp64;
    returns (max [B*H, NC, M], den, num [B*H, NC, M, Dv])."""
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    NC = -(-N // chunk)
    S = scale * np.einsum("bnhd,hmd->bhnm", K, Q)          # [B,H,N,M]
    Vt = V.transpose(0, 2, 1, 3)                            # [B,H,N,Dv]
    mx = np.empty((B, H, NC, M)); den = np.empty((B, H, NC, M)); num = np.empty((B, H, NC, M, Dv))
    for c in range(NC):
        sl = slice(c * chunk, min(N, (c + 1) * chunk))
        m = S[:, :, sl].max(axis=2)
        e = np.exp(S[:, :, sl] - m[:, :, None])
        mx[:, :, c], den[:, :, c] = m, e.sum(axis=2)
        num[:, :, c] = np.einsum("bhtm,bhtd->bhmd", e, Vt[:, :, sl])
    return mx.reshape(B * H, NC, M), den.reshape(B * H, NC, M), num.reshape(B * H, NC, M, Dv)


def stablemax_transform(x, power):
    """The stablemax score transform (stablemax.py:45-52): (1 + x)^p for x >= 0,
    (1 - x)^-p for x < 0.  fp64."""
    x = np.asarray(x, np.float64)
    return np.where(x >= 0, np.power(np.where(x >= 0, 1.0 + x, 1.0), power),
                    np.power(np.where(x < 0, 1.0 - x, 1.0), -power))


def brute_stablemax(Q, K, V, power=2.0, scale=None, Q_dec=None, K_dec=None):
    """Stablemax FLARE by its per-token definition (stablemax_triton.py:1718-1731,
    stablemax.py:595-603): z_t[m] = sum_{tau<=t} s(a_tau,m) v_tau / sum_{tau<=t} s(a_tau,m),
    y_t = sum_m softmax_m(scale qd_t . kd_m) z_t[m].  fp64, one token at a time."""
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    Qd = _f64(Q_dec) if Q_dec is not None else K
    Kd = _f64(K_dec) if K_dec is not None else Q
    W = stablemax_transform(scale * np.einsum("bnhd,hmd->bhnm", K, Q), power)   # [B,H,N,M]
    A = scale * np.einsum("bnhd,hmd->bhnm", Qd, Kd)
    Vt = V.transpose(0, 2, 1, 3)
    Y = np.empty((B, H, N, Dv))
    for t in range(N):
        den = W[:, :, : t + 1].sum(axis=2)                                       # [B,H,M]
        num = np.einsum("bhtm,bhtd->bhmd", W[:, :, : t + 1], Vt[:, :, : t + 1])
        alpha = _softmax(A[:, :, t, :], axis=-1)
        Y[:, :, t] = np.einsum("bhm,bhmd->bhd", alpha, num / den[..., None])
    return Y.transpose(0, 2, 1, 3)


def stablemax_chunked(Q, K, V, power=2.0, scale=None, chunk_size=64, Q_dec=None, K_dec=None):
    """Stablemax FLARE in the chunked form of the reference's PyTorch path
    (stablemax.py:578-635): per-chunk encoder den / num, strict chunk prefixes,
    the decoder softmax over latents, then prefix_out + tril(R W^T) V inside each
    chunk with R = p_dec / total_den.  fp64; a different summation from
    brute_stablemax, against which tests/test_oracle.py pins it."""
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    Qd = _f64(Q_dec) if Q_dec is not None else K
    Kd = _f64(K_dec) if K_dec is not None else Q
    C = int(chunk_size)
    NC = -(-N // C)
    pad = NC * C - N
    Kp = np.concatenate([K, np.zeros((B, pad, H, Dk))], axis=1)
    Vp = np.concatenate([V, np.zeros((B, pad, H, Dv))], axis=1)
    Qdp = np.concatenate([Qd, np.zeros((B, pad, H, Dk))], axis=1)
    Kc = Kp.reshape(B, NC, C, H, Dk).transpose(0, 3, 1, 2, 4)                   # [B,H,NC,C,Dk]
    Vc = Vp.reshape(B, NC, C, H, Dv).transpose(0, 3, 1, 2, 4)
    Qdc = Qdp.reshape(B, NC, C, H, Dk).transpose(0, 3, 1, 2, 4)
    W = stablemax_transform(scale * np.einsum("bhncd,hmd->bhncm", Kc, Q), power)
    if pad:
        W[:, :, -1, C - pad:, :] = 0.0      # padded tokens carry no weight
    cden = W.sum(axis=3)                                                          # [B,H,NC,M]
    cnum = np.einsum("bhncm,bhncd->bhnmd", W, Vc)
    prev_den = np.cumsum(cden, axis=2) - cden
    prev_num = np.cumsum(cnum, axis=2) - cnum
    p_dec = _softmax(scale * np.einsum("bhncd,hmd->bhncm", Qdc, Kd), axis=-1)
    total = prev_den[:, :, :, None, :] + np.cumsum(W, axis=3)
    R = p_dec / np.where(total > 0, total, 1.0)
    prefix_out = np.einsum("bhncm,bhnmd->bhncd", R, prev_num)
    mix = np.einsum("bhncm,bhnsm->bhncs", R, W) * np.tril(np.ones((C, C)))
    Yc = prefix_out + np.einsum("bhncs,bhnsd->bhncd", mix, Vc)
    return Yc.reshape(B, H, NC * C, Dv)[:, :, :N].transpose(0, 2, 1, 3)


def brute_ar_state(Q, K, V, state=None, scale=1.0, attention_mask=None, Q_dec=None, K_dec=None):
    """Prefill continuing a cached state {m,d,u} (inference.py:66-120 semantics), fp64.

    The cached state stands for earlier tokens with weights exp(m) * d (denominator)
    and exp(m) * u (numerator).  Masked tokens contribute nothing and output y = 0
    (inference.py:279-311).  Returns (Y, state) with the state in the convention
    m = running max of all seen scores.
    """
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    H, M, Dk = Q.shape
    B, T, _, Dv = V.shape
    Qd = _f64(Q_dec) if Q_dec is not None else K
    Kd = _f64(K_dec) if K_dec is not None else Q
    valid = np.ones((B, T), bool) if attention_mask is None else (np.asarray(
        attention_mask.cpu() if hasattr(attention_mask, "cpu") else attention_mask) != 0)
    S = scale * np.einsum("bnhd,hmd->bhnm", K, Q)
    A = scale * np.einsum("bnhd,hmd->bhnm", Qd, Kd)
    Vt = V.transpose(0, 2, 1, 3)
    if state is None:
        m0 = np.full((B, H, M), -np.inf)
        d0 = np.zeros((B, H, M))
        u0 = np.zeros((B, H, M, Dv))
    else:
        m0, d0, u0 = _f64(state["m"]), _f64(state["d"]), _f64(state["u"])
    Y = np.zeros((B, H, T, Dv))
    mfin, dfin, ufin = m0.copy(), d0.copy(), u0.copy()
    for b in range(B):
        for h in range(H):
            for t in range(T):
                sel = np.nonzero(valid[b, : t + 1])[0]
                s = S[b, h, sel, :]                              # [n_valid, M]
                mx = np.maximum(m0[b, h], s.max(axis=0) if len(sel) else -np.inf)
                mx_safe = np.where(np.isneginf(mx), 0.0, mx)
                w_state = np.where(np.isneginf(m0[b, h]), 0.0, np.exp(m0[b, h] - mx_safe))
                w_tok = np.exp(s - mx_safe)                      # [n, M]
                den = d0[b, h] * w_state + w_tok.sum(axis=0)
                num = u0[b, h] * w_state[:, None] + w_tok.T @ Vt[b, h, sel]
                if t == T - 1:
                    mfin[b, h], dfin[b, h], ufin[b, h] = mx, den, num
                if not valid[b, t]:
                    continue
                z = num / np.where(den > 0, den, 1.0)[:, None]
                alpha = _softmax(A[b, h, t])
                Y[b, h, t] = alpha @ z
    return Y.transpose(0, 2, 1, 3), {"m": mfin, "d": dfin, "u": ufin}


def brute_semi_ar(Q, K, V, block_size, scale=None, Q_dec=None, K_dec=None):
    """semi_autoregressive/reference.py:560-597: per block, two SDPAs over all tokens < block end. fp64."""
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    Qd = _f64(Q_dec) if Q_dec is not None else K
    Kd = _f64(K_dec) if K_dec is not None else Q
    S = scale * np.einsum("bnhd,hmd->bhnm", K, Q)
    A = scale * np.einsum("bnhd,hmd->bhnm", Qd, Kd)
    Vt = V.transpose(0, 2, 1, 3)
    Y = np.empty((B, H, N, Dv))
    for g in range(math.ceil(N / block_size)):
        t0, t1 = g * block_size, min(N, (g + 1) * block_size)
        P = _softmax(S[:, :, :t1, :], axis=2)
        Z = np.einsum("bhtm,bhtd->bhmd", P, Vt[:, :, :t1])
        alpha = _softmax(A[:, :, t0:t1, :], axis=-1)
        Y[:, :, t0:t1] = np.einsum("bhtm,bhmd->bhtd", alpha, Z)
    return Y.transpose(0, 2, 1, 3)


def brute_semi_ar_state(Q, K, V, block_size, state=None, scale=None, Q_dec=None, K_dec=None):
    """Block-causal FLARE continuing a cached state {m, d, u}, fp64 (semi-AR cached prefill).

    The reference ships no implementation (its semi_autoregressive/inference.py:5-36 are
    stubs); this is the block-level analogue of ``brute_ar_state``: the cached state
    stands for earlier blocks with weights exp(m) d and exp(m) u (inference.py:66-120),
    and every token of block g reads the latent state after the whole block, as in
    ``brute_semi_ar`` (semi_autoregressive/reference.py:560-597).  Returns (Y, state)
    with m the running max of all seen scores.  Pinned in tests/test_oracle.py by
    ``brute_semi_ar`` (no state), by continuation (prefill(a + b) == prefill(b) after
    prefill(a), split at a block end) and by ``brute_ar_state`` (the final state does
    not depend on the blocking).
    """
    Q, K, V = _f64(Q), _f64(K), _f64(V)
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    Qd = _f64(Q_dec) if Q_dec is not None else K
    Kd = _f64(K_dec) if K_dec is not None else Q
    S = scale * np.einsum("bnhd,hmd->bhnm", K, Q)
    A = scale * np.einsum("bnhd,hmd->bhnm", Qd, Kd)
    Vt = V.transpose(0, 2, 1, 3)
    if state is None:
        mc = np.full((B, H, M), -np.inf)
        dc = np.zeros((B, H, M))
        uc = np.zeros((B, H, M, Dv))
    else:
        mc, dc, uc = (_f64(state[k]).copy() for k in ("m", "d", "u"))
    Y = np.zeros((B, H, N, Dv))
    for g in range(math.ceil(N / block_size)):
        t0, t1 = g * block_size, min(N, (g + 1) * block_size)
        s = S[:, :, t0:t1, :]                                     # [B, H, n, M]
        mn = np.maximum(mc, s.max(axis=2))
        mn_safe = np.where(np.isneginf(mn), 0.0, mn)
        w_state = np.where(np.isneginf(mc), 0.0, np.exp(mc - mn_safe))
        w_tok = np.exp(s - mn_safe[:, :, None, :])
        dc = dc * w_state + w_tok.sum(axis=2)
        uc = uc * w_state[..., None] + np.einsum("bhtm,bhtd->bhmd", w_tok, Vt[:, :, t0:t1])
        mc = mn
        z = uc / np.where(dc > 0, dc, 1.0)[..., None]
        alpha = _softmax(A[:, :, t0:t1, :], axis=-1)
        Y[:, :, t0:t1] = np.einsum("bhtm,bhmd->bhtd", alpha, z)
    return Y.transpose(0, 2, 1, 3), {"m": mc, "d": dc, "u": uc}


def allclose_rel(a, b, dtype_name: str):
    """Tolerance used by every parity test.

    ``_common.py:132-137`` gives (rtol, atol) = (1e-5, 1e-5) for fp32 and
    (1e-2, 1e-2) for bf16/fp16; ``_common.py:144-146`` defines
    max_rel_err = max |a-b| / (|b| + atol).
    Returns (max_rel_err, max_abs_err).
    """
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    atol = 1e-5 if dtype_name == "float32" else 1e-2
    if a.size == 0:
        return 0.0, 0.0
    d = np.abs(a - b)
    return float((d / (np.abs(b) + atol)).max()), float(d.max())


# --------------------------------------------------------------------------
# Gradients (fp64 autograd of the definition)
# --------------------------------------------------------------------------

def ar_forward_torch64(Q, K, V, scale=None, Q_dec=None, K_dec=None):
    """The definition of reference.py:15-47 in fp64 torch ops, differentiable.

    z_t = sum_{tau<=t} e^{s_tau} v_tau / sum_{tau<=t} e^{s_tau} is written with
    cumulative sums relative to each latent's sequence-wide max (exact in fp64
    for the score ranges the tests use); y_t = softmax_m(a_t) . z_t.  Inputs
    must be fp64 torch tensors; returns Y [B, N, H, Dv].
    """
    import torch
    H, M, Dk = Q.shape
    scale = resolve_scale(scale, Dk)
    Qd = K if Q_dec is None else Q_dec
    Kd = Q if K_dec is None else K_dec
    S = scale * torch.einsum("bnhd,hmd->bhnm", K, Q)
    A = scale * torch.einsum("bnhd,hmd->bhnm", Qd, Kd)
    E = torch.exp(S - S.amax(dim=2, keepdim=True))                      # [B,H,N,M]
    Vt = V.transpose(1, 2)                                              # [B,H,N,Dv]
    num = torch.cumsum(E.unsqueeze(-1) * Vt.unsqueeze(3), dim=2)        # [B,H,N,M,Dv]
    Z = num / torch.cumsum(E, dim=2).unsqueeze(-1)
    Y = torch.einsum("bhnm,bhnmd->bhnd", torch.softmax(A, dim=-1), Z)
    return Y.transpose(1, 2)


def ar_grads(Q, K, V, dY, scale=None, Q_dec=None, K_dec=None):
    """Gradients of sum(Y * dY) w.r.t. (Q, K, V, Q_dec, K_dec), fp64 autograd --
    the ground truth of the reference's backward tests
    (testing/autoregressive/test_flare.py:184-219, 370-427), which backpropagate
    (y * grad_out).sum() through the torch reference.  Returns numpy arrays
    (None for an absent decoder tensor)."""
    import torch

    def leaf(x):
        return None if x is None else torch.as_tensor(_f64(x)).requires_grad_(True)

    q, k, v, qd, kd = (leaf(x) for x in (Q, K, V, Q_dec, K_dec))
    y = ar_forward_torch64(q, k, v, scale, qd, kd)
    (y * torch.as_tensor(_f64(dY))).sum().backward()
    return tuple(None if x is None else x.grad.numpy() for x in (q, k, v, qd, kd))


def stablemax_forward_torch64(Q, K, V, power=2.0, scale=None, Q_dec=None, K_dec=None):
    """The stablemax definition of brute_stablemax (stablemax_triton.py:1718-1731) in fp64
    torch ops, differentiable: E = s(a) with the piecewise transform, z_t = cumsum(E v) /
    cumsum(E), y_t = softmax_m(scale qd_t . kd_m) . z_t.  Returns Y [B, N, H, Dv]."""
    import torch
    H, M, Dk = Q.shape
    scale = resolve_scale(scale, Dk)
    Qd = K if Q_dec is None else Q_dec
    Kd = Q if K_dec is None else K_dec
    S = scale * torch.einsum("bnhd,hmd->bhnm", K, Q)
    A = scale * torch.einsum("bnhd,hmd->bhnm", Qd, Kd)
    pos = torch.where(S >= 0, S + 1.0, torch.ones_like(S))
    neg = torch.where(S < 0, 1.0 - S, torch.ones_like(S))
    E = torch.where(S >= 0, pos ** power, neg ** (-power))
    Vt = V.transpose(1, 2)
    num = torch.cumsum(E.unsqueeze(-1) * Vt.unsqueeze(3), dim=2)
    Z = num / torch.cumsum(E, dim=2).unsqueeze(-1)
    Y = torch.einsum("bhnm,bhnmd->bhnd", torch.softmax(A, dim=-1), Z)
    return Y.transpose(1, 2)


def stablemax_grads(Q, K, V, dY, power=2.0, scale=None, Q_dec=None, K_dec=None):
    """Gradients of sum(Y * dY) for the stablemax forward, fp64 autograd -- the ground
    truth of the reference's stablemax backward test (testing/autoregressive/
    test_stablemax.py, backward against the PyTorch path).  Returns numpy arrays
    (None for an absent decoder tensor)."""
    import torch

    def leaf(x):
        return None if x is None else torch.as_tensor(_f64(x)).requires_grad_(True)

    q, k, v, qd, kd = (leaf(x) for x in (Q, K, V, Q_dec, K_dec))
    y = stablemax_forward_torch64(q, k, v, power, scale, qd, kd)
    (y * torch.as_tensor(_f64(dY))).sum().backward()
    return tuple(None if x is None else x.grad.numpy() for x in (q, k, v, qd, kd))


def semi_forward_torch64(Q, K, V, block_size, scale=None, Q_dec=None, K_dec=None):
    """Block-causal definition (semi_autoregressive/reference.py:560-597: token t of
    block g attends to every token of blocks <= g) in fp64 torch ops: the
    cumulative sums of ar_forward_torch64 read at each block's last token."""
    import torch
    H, M, Dk = Q.shape
    B, N, _, Dv = V.shape
    scale = resolve_scale(scale, Dk)
    Qd = K if Q_dec is None else Q_dec
    Kd = Q if K_dec is None else K_dec
    S = scale * torch.einsum("bnhd,hmd->bhnm", K, Q)
    A = scale * torch.einsum("bnhd,hmd->bhnm", Qd, Kd)
    E = torch.exp(S - S.amax(dim=2, keepdim=True))
    Vt = V.transpose(1, 2)
    num = torch.cumsum(E.unsqueeze(-1) * Vt.unsqueeze(3), dim=2)
    Z = num / torch.cumsum(E, dim=2).unsqueeze(-1)                      # [B,H,N,M,Dv]
    ends = (torch.arange(N) // block_size + 1) * block_size - 1         # each token's block end
    Y = torch.einsum("bhnm,bhnmd->bhnd", torch.softmax(A, dim=-1), Z[:, :, ends])
    return Y.transpose(1, 2)


def semi_grads(Q, K, V, dY, block_size, scale=None, Q_dec=None, K_dec=None):
    """Gradients of sum(Y * dY) for the block-causal forward, fp64 autograd --
    the ground truth of the reference's block-causal backward tests
    (testing/semi_autoregressive/test_block_causal.py:346-578)."""
    import torch

    def leaf(x):
        return None if x is None else torch.as_tensor(_f64(x)).requires_grad_(True)

    q, k, v, qd, kd = (leaf(x) for x in (Q, K, V, Q_dec, K_dec))
    y = semi_forward_torch64(q, k, v, block_size, scale, qd, kd)
    (y * torch.as_tensor(_f64(dY))).sum().backward()
    return tuple(None if x is None else x.grad.numpy() for x in (q, k, v, qd, kd))
