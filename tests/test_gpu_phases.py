"""GPU parity of the chunked forward's phase entry points through the C ABI:
flare_chunk_prepare (chunk_prepare_tr on the MFMA shapes, the fp32 kernel
otherwise) against the fp64 chunk summaries of the oracle (``chunk_summaries``,
pinned in tests/test_oracle.py), and flare_chunk_prefix against the exclusive
online-softmax scan of those summaries (reference training.py:914-1103).

Summaries are compared with the row-wise state bar of tests/_util.py
(assert_state_rowwise)."""
import sys

import numpy as np
import pytest
import torch

import flare_oracle as O
from _util import assert_state_rowwise as assert_summary_parity, seeded, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(*args):
    print("CASE", *args, flush=True)
    sys.stdout.flush()


def _prepare(q, k, v, chunk, scale):
    from causal_flare import _lib
    lib = _lib.lib()
    B, N, H, D = v.shape
    M = q.shape[1]
    NC = -(-N // chunk)
    cmax = torch.empty((B * H, NC, M), device=DEV)
    cden = torch.empty_like(cmax)
    cnum = torch.empty((B * H, NC, M, D), device=DEV)
    P = _lib.ptr
    rc = lib.flare_chunk_prepare(P(q), P(k), P(v), _lib.dtype_code(q.dtype), B, N, H, M, q.shape[2], D, float(scale),
                                 chunk, P(cmax), P(cden), P(cnum), _lib.stream_of(q.device))
    _lib.check(rc, "flare_chunk_prepare")
    return cmax, cden, cnum


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,D,N,chunk", [(256, 128, 1100, 512), (128, 64, 1000, 96), (256, 64, 777, 256),
                                         (128, 128, 300, 64)])
def test_chunk_prepare_summaries(dtype, M, D, N, chunk):
    """Ragged lengths, chunks that are not whole 64-token tiles (96) and a last tile
    that ends inside the chunk; max in natural-log units, den and num relative to it."""
    _case("chunk_prepare", dtype, M, D, N, chunk)
    B, H = 2, 2
    q, k, v = seeded(80 + M + D, B, N, H, M, D, D, dtype, q_std=D ** -0.5)
    scale = D ** -0.5
    cmax, cden, cnum = _prepare(q.to(DEV), k.to(DEV), v.to(DEV), chunk, scale)
    mx, den, num = O.chunk_summaries(q, k, v, chunk, scale=scale)
    assert_summary_parity((cmax, cden, cnum), (mx, den, num), dtype, f"prepare {dtype} M={M} D={D} N={N} chunk={chunk}")


def test_chunk_prepare_values_outside_fp16():
    """bf16 V far outside the fp16 range in some chunks: the prepare kernel's fp16 pass
    meets an inf and redoes those chunks with bf16 hi + lo weights against bf16 V."""
    _case("chunk_prepare large values")
    B, N, H, M, D, chunk = 1, 2048, 2, 256, 128, 512
    q, k, v = seeded(88, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    v = v.float()
    v[:, 600:610] *= 2e5
    v[:, 1500, 1] = 1e30
    v = v.bfloat16()
    cmax, cden, cnum = _prepare(q.to(DEV), k.to(DEV), v.to(DEV), chunk, D ** -0.5)
    mx, den, num = O.chunk_summaries(q, k, v, chunk, scale=D ** -0.5)
    assert_summary_parity((cmax, cden, cnum), (mx, den, num), torch.bfloat16, "prepare with values outside fp16")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_chunk_prefix_scan(dtype):
    """flare_chunk_prefix overwrites the summaries with exclusive prefixes: chunk c's
    entry is the merge of chunks 0 .. c-1 (chunk 0: max -inf, den 0, num 0)."""
    from causal_flare import _lib
    _case("chunk_prefix", dtype)
    B, N, H, M, D, chunk = 2, 900, 2, 128, 64, 128
    q, k, v = seeded(89, B, N, H, M, D, D, dtype, q_std=D ** -0.5)
    cmax, cden, cnum = _prepare(q.to(DEV), k.to(DEV), v.to(DEV), chunk, D ** -0.5)
    lib = _lib.lib()
    NC = cmax.shape[1]
    rc = lib.flare_chunk_prefix(_lib.ptr(cmax), _lib.ptr(cden), _lib.ptr(cnum), B * H, NC, M, D,
                                None, None, None, None, None, None, _lib.stream_of(cmax.device))
    _lib.check(rc, "flare_chunk_prefix")
    mx, den, num = O.chunk_summaries(q, k, v, chunk, scale=D ** -0.5)
    pm, pd, pn = to_np(cmax), to_np(cden), to_np(cnum)
    assert np.isneginf(pm[:, 0]).all() and (pd[:, 0] == 0).all() and (pn[:, 0] == 0).all()
    m, d, u = mx[:, 0], den[:, 0], num[:, 0]
    for c in range(1, NC):
        assert_summary_parity((cmax[:, c], cden[:, c], cnum[:, c]), (m, d, u), dtype, f"prefix chunk {c}")
        mn = np.maximum(m, mx[:, c])
        a, b = np.exp(m - mn), np.exp(mx[:, c] - mn)
        d, u, m = d * a + den[:, c] * b, u * a[..., None] + num[:, c] * b[..., None], mn
