"""GPU parity of the semi-autoregressive cached prefill and block decode
(flare_semi_autoregressive_prefill_trition / _decode_trition, C entry point
flare_semi_ar_forward_state) against the fp64 oracle ``brute_semi_ar_state``.

The reference has no implementation of these entry points (stubs in
causal_flare/semi_autoregressive/inference.py:5-36); the oracle is the block-level
analogue of its cached prefill (autoregressive/inference.py:231-315) and is pinned
in tests/test_oracle.py.  Tolerances: tests/_util.py (assert_parity,
assert_state_parity).
"""
import sys

import numpy as np
import pytest
import torch

import flare_oracle as O
from _util import assert_parity, assert_state_parity, seeded, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(*args):
    print("CASE", *args, flush=True)
    sys.stdout.flush()


def _cached_state(B, T, H, M, D, dtype, seed=40):
    """A cache left by the autoregressive prefill of T random tokens (on the GPU)."""
    import causal_flare
    q, k, v = seeded(seed, B, T, H, M, D, D, dtype, q_std=D ** -0.5)
    _, st = causal_flare.flare_autoregressive_prefill_triton(q.to(DEV), k.to(DEV), v.to(DEV))
    return q, st


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,N,H,M,D,block", [(2, 256, 4, 128, 64, 64), (1, 192, 2, 64, 32, 32), (1, 128, 2, 256, 128, 128)])
def test_semi_prefill_with_state(dtype, B, N, H, M, D, block):
    import causal_flare
    _case("semi prefill state", dtype, B, N, H, M, D, block)
    q, st = _cached_state(B, 96, H, M, D, dtype)
    _, k, v = seeded(41, B, N, H, M, D, D, dtype, q_std=D ** -0.5)
    y, st_out = causal_flare.flare_semi_autoregressive_prefill_trition(
        q.to(DEV), k.to(DEV), v.to(DEV), state=st, block_size=block)
    ref_st = {key: to_np(st[key]) for key in ("m", "d", "u")}
    yr, str_ = O.brute_semi_ar_state(q, k, v, block, state=ref_st)
    assert_parity(y, yr, dtype, "semi prefill with state")
    assert_state_parity(st_out, str_, dtype, "semi prefill")
    # the input state is left untouched
    assert st_out["m"].data_ptr() != st["m"].data_ptr()


def test_semi_prefill_without_state_is_the_block_causal_forward():
    import causal_flare
    _case("semi prefill no state")
    B, N, H, M, D, block = 2, 512, 4, 128, 64, 64
    q, k, v = seeded(42, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    y, st = causal_flare.flare_semi_autoregressive_prefill_trition(qd, kd, vd, block_size=block)
    yf, _ = causal_flare.flare_semi_autoregressive_trition(qd, kd, vd, block_size=block, chunk_size=64)
    assert torch.equal(y, yf)
    yr, str_ = O.brute_semi_ar_state(q, k, v, block)
    assert_parity(y, yr, torch.bfloat16, "semi prefill")
    assert_state_parity(st, str_, torch.bfloat16, "semi prefill")


def test_semi_prefill_continuation_cfg5():
    """Config 5 (B=2, N=8192, H=16, M=128, D=64, block 64): two prefills of 4096 tokens,
    the second from the first's state, equal the block-causal forward over all 8192."""
    import causal_flare
    _case("semi prefill continuation cfg5")
    B, N, H, M, D, block = 2, 8192, 16, 128, 64, 64
    q, k, v = seeded(4, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    cut = N // 2
    y1, st = causal_flare.flare_semi_autoregressive_prefill_trition(qd, kd[:, :cut], vd[:, :cut], block_size=block)
    y2, st2 = causal_flare.flare_semi_autoregressive_prefill_trition(qd, kd[:, cut:], vd[:, cut:], state=st,
                                                                    block_size=block)
    y = torch.cat([y1, y2], dim=1)
    ref, _, _ = O.semi_ar(q, k, v, block, 64, nthreads=16)
    assert_parity(y, ref, torch.bfloat16, "cfg5 continued")
    _, st_ar = O.ar_recurrent(q, k, v, scale=D ** -0.5, nthreads=16)
    assert_state_parity(st2, st_ar, torch.bfloat16, "cfg5 final state")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_semi_decode_block_in_place(dtype):
    import causal_flare
    _case("semi decode", dtype)
    B, H, M, D, T = 3, 4, 128, 64, 32
    q, st = _cached_state(B, 70, H, M, D, dtype)
    ref_st = {key: to_np(st[key]) for key in ("m", "d", "u")}
    ptrs = {key: st[key].data_ptr() for key in st}
    for step in range(3):
        _, k, v = seeded(50 + step, B, T, H, M, D, D, dtype)
        y, st_ret = causal_flare.flare_semi_autoregressive_decode_trition(q.to(DEV), k.to(DEV), v.to(DEV), state=st)
        yr, ref_st = O.brute_semi_ar_state(q, k, v, T, state=ref_st)
        assert_parity(y, yr, dtype, f"semi decode step {step}")
        assert all(st_ret[key].data_ptr() == ptrs[key] for key in st)   # updated in place
    assert_state_parity(st, ref_st, dtype, "semi decode state")


def test_semi_decode_single_token_is_autoregressive_step():
    import causal_flare
    _case("semi decode one token")
    B, H, M, D = 2, 4, 64, 32
    q, st = _cached_state(B, 40, H, M, D, torch.bfloat16)
    st2 = {key: t.clone() for key, t in st.items()}
    _, k, v = seeded(60, B, 1, H, M, D, D, torch.bfloat16)
    y, _ = causal_flare.flare_semi_autoregressive_decode_trition(q.to(DEV), k[:, 0].to(DEV), v[:, 0].to(DEV),
                                                                state=st)
    ya, _ = causal_flare.flare_autoregressive_decode_triton(q.to(DEV), k[:, 0].to(DEV), v[:, 0].to(DEV), state=st2,
                                                          scale=D ** -0.5)
    assert torch.equal(y, ya)
    assert all(torch.equal(st[key], st2[key]) for key in st)


def test_semi_prefill_separate_decoder_with_state():
    import causal_flare
    _case("semi prefill separate decoder")
    B, N, H, M, D, block = 2, 128, 2, 128, 64, 32
    q, st = _cached_state(B, 50, H, M, D, torch.bfloat16)
    g = torch.Generator().manual_seed(61)
    _, k, v = seeded(62, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    qdec = torch.randn(k.shape, generator=g).to(torch.bfloat16)
    kdec = (torch.randn(q.shape, generator=g) * D ** -0.5).to(torch.bfloat16)
    y, st_out = causal_flare.flare_semi_autoregressive_prefill_trition(
        q.to(DEV), k.to(DEV), v.to(DEV), state=st, block_size=block, Q_dec=qdec.to(DEV), K_dec=kdec.to(DEV))
    ref_st = {key: to_np(st[key]) for key in ("m", "d", "u")}
    yr, str_ = O.brute_semi_ar_state(q, k, v, block, state=ref_st, Q_dec=qdec, K_dec=kdec)
    assert_parity(y, yr, torch.bfloat16, "semi prefill separate decoder")
    assert_state_parity(st_out, str_, torch.bfloat16, "semi prefill separate decoder")
