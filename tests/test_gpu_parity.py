"""GPU parity: the HIP kernels (through the drop-in Python entry points and the
C ABI) against the fp32 CPU oracle on identical seeded inputs.

Mirrors the reference's GPU suites: testing/autoregressive/test_flare.py:342-490
(chunked / prefill / decode parity, 3x3 decoder-aliasing modes),
testing/autoregressive/test_cached_suites.py:24-104 (masked prefill, decode
continuation) and testing/semi_autoregressive/test_block_causal.py:178-255.
Tolerances are stated in tests/_util.py (assert_parity).
"""
import math
import sys

import numpy as np
import pytest
import torch

import flare_oracle as O
from _util import assert_noise_model, assert_parity, assert_state_parity, assert_state_rowwise, seeded, to_np

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _print_case(*args):
    print("CASE", *args, flush=True)
    sys.stdout.flush()


def _dec_variants(q, k, g):
    qd_rand = torch.randn(k.shape, generator=g).to(k.dtype).to(k.device)
    kd_rand = torch.randn(q.shape, generator=g).to(q.dtype).to(q.device)
    return {"none": None, "k_enc": k, "rand": qd_rand}, {"none": None, "q_enc": q, "rand": kd_rand}


def _oracle_dec(x, enc):
    """The oracle takes None for the default decoder tensor."""
    return None if (x is None or x is enc) else x


# --------------------------------------------------------------------------
# Full-sequence chunked forward
# --------------------------------------------------------------------------
@pytest.mark.parametrize("d_score,d_value", [(16, 16), (64, 128)])
def test_chunked_forward_decoder_variants_fp32(d_score, d_value):
    from causal_flare import flare_autoregressive_triton
    B, N, H, M = 1, 16, 2, 16
    _print_case("chunked_fp32_variants", d_score, d_value)
    q, k, v = seeded(2028, B, N, H, M, d_score, d_value, torch.float32, device=DEV)
    g = torch.Generator().manual_seed(7)
    qds, kds = _dec_variants(q, k, g)
    scale = 1.0 / math.sqrt(d_score)
    for qn, qd in qds.items():
        for kn, kd in kds.items():
            y = flare_autoregressive_triton(q, k, v, scale=scale, chunk_size=16, Q_dec=qd, K_dec=kd)
            ref = O.ar_chunked(q, k, v, scale=scale, chunk_size=16, Q_dec=_oracle_dec(qd, k),
                               K_dec=_oracle_dec(kd, q))
            assert y.dtype == torch.float32
            assert_parity(y, ref, torch.float32, f"chunked q_dec={qn} k_dec={kn}")


@pytest.mark.parametrize("chunk", [None, 16, 48, 64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chunked_forward_ragged_lengths(chunk, dtype):
    from causal_flare import flare_autoregressive_triton
    B, N, H, M, D = 2, 203, 3, 32, 64
    _print_case("chunked_ragged", chunk, dtype)
    q, k, v = seeded(11, B, N, H, M, D, D, dtype, q_std=D ** -0.5, device=DEV)
    y = flare_autoregressive_triton(q, k, v, chunk_size=chunk)
    assert y.dtype == dtype
    ref = O.ar_chunked(q, k, v)
    assert_parity(y, ref, dtype, f"ragged chunk={chunk}")


def test_cfg1_cpu_reference_shape_fp32():
    """B=1, N=256, H=8, M=64, D=32, fp32, q ~ N(0,1), seed 0."""
    from causal_flare import flare_autoregressive_triton
    _print_case("cfg1")
    torch.manual_seed(0)
    q = torch.randn(8, 64, 32)
    k = torch.randn(1, 256, 8, 32)
    v = torch.randn(1, 256, 8, 32)
    y = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV))
    assert_parity(y, O.ar_chunked(q, k, v), torch.float32, "cfg1")
    # and against the fp64 two-SDPA definition itself
    assert_parity(y, O.brute_ar(q, k, v), torch.float32, "cfg1 brute")


def _cfg_inputs(seed, B, N, H, M, D, dtype):
    torch.manual_seed(seed)
    q = torch.randn(H, M, D) / math.sqrt(D)
    k = torch.randn(B, N, H, D)
    v = torch.randn(B, N, H, D)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def test_cfg2_chunked_prefill_bf16():
    """B=4, N=4096, H=16, M=128, D=64, bf16, seed 1."""
    from causal_flare import flare_autoregressive_triton
    _print_case("cfg2")
    q, k, v = _cfg_inputs(1, 4, 4096, 16, 128, 64, torch.bfloat16)
    y = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV))
    assert y.dtype == torch.bfloat16
    ref = O.ar_chunked(q, k, v, nthreads=16)
    assert_parity(y, ref, torch.bfloat16, "cfg2")


def test_cfg3_long_context_bf16():
    """BASELINE config 3 (B=1, N=65536, H=16, M=256, D=128, bf16, seed 2): every
    head against the oracle at full length."""
    from causal_flare import flare_autoregressive_triton
    _print_case("cfg3")
    q, k, v = _cfg_inputs(2, 1, 65536, 16, 256, 128, torch.bfloat16)
    y = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    ref = O.ar_chunked(q, k, v, scale=128 ** -0.5, nthreads=16)
    assert_parity(y, ref, torch.bfloat16, "cfg3 all heads")


def _jump_keys(q, k, tokens, lat, nats, scale):
    """Key outliers: at tokens[i], the key of every head points along the sum of the
    latent directions `lat`, scaled so that the smallest of those latents' scores is
    nats[i]; their references jump by far more than the fp32 range covers within
    one 32-token subtile."""
    k = k.clone().float()
    qf = q.float()
    for h in range(q.shape[0]):
        u = sum(qf[h, m] / qf[h, m].norm() for m in lat)
        s = torch.stack([qf[h, m] @ u for m in lat]).min() * scale
        for t, n in zip(tokens, nats):
            k[:, t, h] = u * (n / float(s))
    return k.to(q.dtype)


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_score_jump_within_subtile(M, D, dtype):
    """A latent whose score jumps by ~150 nats in the middle of a 32-token subtile
    (one in chunk 0 with no reference yet, one deep in a later chunk): the earlier
    tokens of that subtile must keep the latent, as in the tokenwise recurrence
    (training.py:1351-1371).  The MFMA output kernel flags such chunks and the
    tokenwise fp32 kernel replays them."""
    from causal_flare import flare_autoregressive_triton
    _print_case("score_jump", M, D, dtype)
    B, N, H = 2, 1100, 2
    q, k, v = seeded(404 + M, B, N, H, M, D, D, dtype, q_std=D ** -0.5)
    scale = D ** -0.5
    lat = list(range(0, M, M // 8))
    kj = _jump_keys(q, k, [17, 256 + 3 * 32 + 17, 900 + 9], lat=lat, nats=[150.0, 300.0, 450.0], scale=scale)
    ref = O.ar_chunked(q, kj, v, scale=scale, nthreads=16)
    for chunk in (None, 256):
        y = flare_autoregressive_triton(q.to(DEV), kj.to(DEV), v.to(DEV), chunk_size=chunk)
        assert_parity(y, ref, dtype, f"score jump M={M} D={D} chunk={chunk}")
    # The same outlier key three times: the later two do not move the reference
    # (their scores equal the latents' running max), so those chunks stay on the MFMA
    # kernel, where one latent takes nearly all of a token's decoder weight and its z
    # averages a few O(1) values: the sharp-softmax regime, held to the reference
    # suite's bf16 noise-model bar (fp16 readout operands, |error| ~ 2e-4 here).
    kr = _jump_keys(q, k, [17, 256 + 3 * 32 + 17, 900 + 9], lat=lat, nats=[150.0] * 3, scale=scale)
    ref = O.ar_chunked(q, kr, v, scale=scale, nthreads=16)
    y = flare_autoregressive_triton(q.to(DEV), kr.to(DEV), v.to(DEV))
    assert_noise_model(y, ref, f"repeated outlier M={M} D={D}")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
def test_score_jump_in_ragged_tail(M, D):
    """A jump in the last, partial subtile of the sequence (N = 1100: the default chunk
    leaves a 12-token last chunk, chunk 256 a 76-token one whose third subtile holds 12
    tokens): the replay of the flagged subtile stops at the sequence end."""
    from causal_flare import flare_autoregressive_triton
    _print_case("score_jump_tail", M, D)
    B, N, H = 1, 1100, 2
    q, k, v = seeded(505 + M, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    scale = D ** -0.5
    lat = list(range(0, M, M // 8))
    kj = _jump_keys(q, k, [1090, 1097], lat=lat, nats=[200.0, 350.0], scale=scale)
    ref = O.ar_chunked(q, kj, v, scale=scale, nthreads=16)
    for chunk in (None, 256):
        y = flare_autoregressive_triton(q.to(DEV), kj.to(DEV), v.to(DEV), chunk_size=chunk)
        assert_parity(y, ref, torch.bfloat16, f"tail jump M={M} D={D} chunk={chunk}")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128), (128, 128), (256, 64)])
def test_score_jumps_replay_flagged_subtiles(M, D):
    """Two jumps in one chunk (subtiles 2 and 5 of a 512-token chunk) and one in the
    first subtile of another chunk: the output kernel records the state at the first
    flagged subtile's start over the chunk's prefix slot, and the tokenwise fp32 replay
    covers subtiles 2 .. 5 (and 0 .. 0) only, from that state -- inside chunk_output_tr
    for the 128 x 64 and 256 x 128 banks, by the replay launch after it for 128 x 128 and
    256 x 64.  Tokens after the replayed range come from the MFMA kernel with the jumped
    references."""
    from causal_flare import flare_autoregressive_triton
    _print_case("score_jump_narrow", M, D)
    B, N, H = 1, 2048, 2
    q, k, v = seeded(808 + M, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    scale = D ** -0.5
    lat = list(range(0, M, M // 8))
    kj = _jump_keys(q, k, [512 + 64 + 5, 512 + 160 + 20, 1536 + 3], lat=lat, nats=[150.0, 300.0, 450.0],
                    scale=scale)
    ref = O.ar_chunked(q, kj, v, scale=scale, nthreads=16)
    y = flare_autoregressive_triton(q.to(DEV), kj.to(DEV), v.to(DEV), chunk_size=512)
    assert_parity(y, ref, torch.bfloat16, f"narrow replay M={M} D={D}")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
@pytest.mark.parametrize("nats", [4.0, 7.5, 8.8, 12.0])
@pytest.mark.parametrize("tok", [9, 100])
def test_key_outlier_spreads_references(M, D, nats, tok):
    """A key at token `tok` sits `nats` above the others on 8 latents (and far off on
    many more), so the latents' references then span up to ~45 powers of two within
    one producer wave: the per-token softmax partials must keep every latent (they
    are summed in fp32), and at token 9 the first subtile of a sequence with no state
    starts its references at that subtile's log-sum-exp only when every E is at least
    2^-12.  Against the tokenwise recurrence (training.py:1282-1393) for the AR path
    and the block-causal forward (semi reference.py:308-536) for the semi-AR path."""
    from causal_flare import flare_autoregressive_triton, flare_semi_autoregressive_trition
    _print_case("key_outlier", M, D, nats, tok)
    B, N, H = 2, 300, 2
    q, k, v = seeded(505 + M, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    scale = D ** -0.5
    kj = _jump_keys(q, k, [tok], lat=list(range(0, M, M // 8)), nats=[nats], scale=scale)
    ref = O.ar_chunked(q, kj, v, scale=scale, nthreads=16)
    for chunk in (None, 64):
        y = flare_autoregressive_triton(q.to(DEV), kj.to(DEV), v.to(DEV), chunk_size=chunk)
        assert_parity(y, ref, torch.bfloat16, f"key outlier M={M} D={D} nats={nats} tok={tok} chunk={chunk}")
    ys, _ = flare_semi_autoregressive_trition(q.to(DEV), kj[:, :288].to(DEV), v[:, :288].to(DEV), block_size=96,
                                              chunk_size=32)
    refs, _, _ = O.semi_ar(q, kj[:, :288], v[:, :288], 96, 32)
    assert_parity(ys, refs, torch.bfloat16, f"semi key outlier M={M} D={D} nats={nats} tok={tok}")


def test_meeting_timeout_falls_back_to_tokenwise_replay():
    """The producer meeting of the output kernel is a bounded wait.  With the bound
    forced to zero from the host, waits give up: the kernel counts the faults and
    flags the chunks, and the tokenwise fp32 replay still gives the right output."""
    from causal_flare import _lib, flare_autoregressive_triton
    _print_case("meet_timeout")
    q, k, v = seeded(31, 2, 1000, 2, 128, 64, 64, torch.bfloat16, q_std=64 ** -0.5)
    ref = O.ar_chunked(q, k, v, nthreads=16)
    _lib.device_faults(reset=True)
    _lib.set_meet_spin_limit(0)
    try:
        y = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV), chunk_size=256)
        faults = _lib.device_faults(reset=True)
    finally:
        _lib.set_meet_spin_limit(1 << 20)
    assert_parity(y, ref, torch.bfloat16, "forced meeting timeouts")
    assert faults > 0, "a zero spin limit should make some producer give up"
    y2 = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV), chunk_size=256)
    assert _lib.device_faults() == 0, "no faults with the default bound"
    assert_parity(y2, ref, torch.bfloat16, "default bound")


def test_score_jump_prefill_with_state_bf16():
    """The same jump in a prefill continued from a cached state, with a token mask."""
    from causal_flare import flare_autoregressive_prefill_triton
    _print_case("score_jump_prefill")
    B, T, H, M, D = 2, 700, 2, 128, 64
    q, k, v = seeded(77, B, 2 * T, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    k = _jump_keys(q, k, [T + 40 + 17, T + 500 + 5], lat=list(range(0, M, 16)), nats=[150.0, 300.0], scale=1.0)
    _, st = flare_autoregressive_prefill_triton(q.to(DEV), k[:, :T].to(DEV), v[:, :T].to(DEV))
    _, st_o = O.ar_recurrent(q, k[:, :T], v[:, :T], nthreads=16)
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[1, 30:50] = 0
    y, st2 = flare_autoregressive_prefill_triton(q.to(DEV), k[:, T:].to(DEV), v[:, T:].to(DEV), state=st,
                                                 attention_mask=mask.to(DEV))
    y_ref, st_ref = O.ar_recurrent(q, k[:, T:], v[:, T:], state=st_o, attention_mask=mask, nthreads=16)
    assert_parity(y, y_ref, torch.bfloat16, "score jump prefill")
    assert_state_parity(st2, st_ref, torch.bfloat16, "score jump prefill")


# --------------------------------------------------------------------------
# Prefill / decode
# --------------------------------------------------------------------------
@pytest.mark.parametrize("q_dec_mode", ["none", "k_enc", "rand"])
@pytest.mark.parametrize("k_dec_mode", ["none", "q_enc", "rand"])
@pytest.mark.parametrize("d_score,d_value", [(16, 16), (64, 128)])
def test_prefill_decode_variants_fp32(q_dec_mode, k_dec_mode, d_score, d_value):
    from causal_flare import flare_autoregressive_decode_triton, flare_autoregressive_prefill_triton
    _print_case("prefill_decode", q_dec_mode, k_dec_mode, d_score, d_value)
    B, N, H, M = 1, 16, 2, 16
    q, k, v = seeded(1337, B, N, H, M, d_score, d_value, torch.float32, device=DEV)
    g = torch.Generator().manual_seed(3)
    qds, kds = _dec_variants(q, k, g)
    qd, kd = qds[q_dec_mode], kds[{"none": "none", "q_enc": "q_enc", "rand": "rand"}[k_dec_mode]]
    scale = 1.0 / math.sqrt(d_score)
    y, st = flare_autoregressive_prefill_triton(Q=q, K=k, V=v, Q_dec=qd, K_dec=kd, scale=scale)
    y_ref, st_ref = O.ar_recurrent(q, k, v, scale=scale, Q_dec=_oracle_dec(qd, k), K_dec=_oracle_dec(kd, q))
    assert_parity(y, y_ref, torch.float32, "prefill y")
    for key in ("m", "d", "u"):
        assert_parity(st[key], st_ref[key], torch.float32, f"prefill state {key}")

    k_next = torch.randn((B, 1, H, d_score), generator=g).to(DEV)
    v_next = torch.randn((B, 1, H, d_value), generator=g).to(DEV)
    qd_next = {"none": None, "k_enc": k_next, "rand": torch.randn((B, 1, H, d_score), generator=g).to(DEV)}[q_dec_mode]
    y1, st1 = flare_autoregressive_decode_triton(Q=q, K=k_next, V=v_next, state=st, Q_dec=qd_next, K_dec=kd,
                                                 scale=scale)
    assert st1["u"] is st["u"], "decode must update the fp32 state in place"
    y1_ref, st1_ref = O.ar_recurrent(q, k_next, v_next, state=st_ref, scale=scale,
                                     Q_dec=_oracle_dec(qd_next, k_next), K_dec=_oracle_dec(kd, q))
    assert y1.shape == (B, 1, H, d_value)
    assert_parity(y1, y1_ref, torch.float32, "decode y")
    for key in ("m", "d", "u"):
        assert_parity(st1[key], st1_ref[key], torch.float32, f"decode state {key}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_decode_continuation_equals_prefill_of_concatenation(dtype):
    """test_cached_suites.py:55-63: prefill(T) + decode steps == prefill(T + steps)."""
    from causal_flare import flare_autoregressive_decode_triton, flare_autoregressive_prefill_triton
    _print_case("continuation", dtype)
    B, T, S, H, M, D = 3, 150, 5, 2, 32, 64
    q, k, v = seeded(5, B, T + S, H, M, D, D, dtype, q_std=D ** -0.5, device=DEV)
    y_all, st_all = flare_autoregressive_prefill_triton(q, k, v)
    y_pre, st = flare_autoregressive_prefill_triton(q, k[:, :T], v[:, :T])
    ys = [y_pre]
    for t in range(T, T + S):
        y_t, st = flare_autoregressive_decode_triton(q, k[:, t:t + 1], v[:, t:t + 1], state=st)
        ys.append(y_t)
    y_cat = torch.cat(ys, dim=1)
    assert_parity(y_cat.float(), y_all.float(), dtype, "continuation y")
    ref, st_ref = O.ar_recurrent(q, k, v)
    assert_parity(y_all, ref, dtype, "prefill vs oracle")
    assert_state_parity(st, st_ref, dtype, "continued")


def test_prefill_with_initial_state_and_mask():
    from causal_flare import flare_autoregressive_prefill_triton
    _print_case("prefill_state_mask")
    B, T, H, M, D = 2, 40, 2, 16, 32
    q, k, v = seeded(9, B, 2 * T, H, M, D, D, torch.float32, device=DEV)
    _, st = flare_autoregressive_prefill_triton(q, k[:, :T], v[:, :T])
    st_keep = {kk: vv.clone() for kk, vv in st.items()}
    y, st2 = flare_autoregressive_prefill_triton(q, k[:, T:], v[:, T:], state=st)
    for kk in st_keep:
        assert torch.equal(st_keep[kk], st[kk]), "prefill must not modify its input state"
    _, st_o = O.ar_recurrent(q, k[:, :T], v[:, :T])
    y_ref, st2_ref = O.ar_recurrent(q, k[:, T:], v[:, T:], state=st_o)
    assert_parity(y, y_ref, torch.float32, "prefill with state")
    assert_parity(st2["u"], st2_ref["u"], torch.float32, "state u")
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[0, 3] = 0
    mask[1, 10:20] = 0
    ym, stm = flare_autoregressive_prefill_triton(q, k[:, T:], v[:, T:], state=st, attention_mask=mask.to(DEV))
    ym_ref, stm_ref = O.ar_recurrent(q, k[:, T:], v[:, T:], state=st_o, attention_mask=mask)
    assert_parity(ym, ym_ref, torch.float32, "masked prefill")
    assert float(ym[0, 3].abs().max()) == 0.0 and float(ym[1, 10:20].abs().max()) == 0.0
    assert_parity(stm["m"], stm_ref["m"], torch.float32, "masked state m")
    assert_parity(stm["u"], stm_ref["u"], torch.float32, "masked state u")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
@pytest.mark.parametrize("with_state", [False, True])
def test_masked_prefill_mfma_bf16(M, D, with_state):
    """Masked prefill on the bf16 MFMA kernels: the first 40 tokens masked (so a
    chunk starts with no reference), scattered tokens, a whole chunk and a chunk
    boundary; against the reference's token-by-token decode semantics
    (inference.py:663-695) restated in the oracle."""
    from causal_flare import flare_autoregressive_prefill_triton
    _print_case("masked_prefill_mfma", M, D, with_state)
    B, T, H = 2, 1100, 2
    q, k, v = seeded(97 + M, B, 2 * T, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    st = st_o = None
    if with_state:
        _, st = flare_autoregressive_prefill_triton(q.to(DEV), k[:, :T].to(DEV), v[:, :T].to(DEV))
        _, st_o = O.ar_recurrent(q, k[:, :T], v[:, :T], nthreads=16)
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[:, :40] = 0
    mask[0, 100:103] = 0
    mask[1, 256:512] = 0
    mask[1, 700:760] = 0
    mask[0, T - 1] = 0
    y, st2 = flare_autoregressive_prefill_triton(q.to(DEV), k[:, T:].to(DEV), v[:, T:].to(DEV), state=st,
                                                 attention_mask=mask.to(DEV))
    y_ref, st_ref = O.ar_recurrent(q, k[:, T:], v[:, T:], state=st_o, attention_mask=mask, nthreads=16)
    assert torch.all(y[mask == 0].float() == 0), "masked tokens must give y = 0"
    assert_parity(y, y_ref, torch.bfloat16, f"masked prefill M={M} D={D} state={with_state}")
    assert_state_parity(st2, st_ref, torch.bfloat16, "masked prefill")


def test_masked_prefill_leading_tokens_fp32():
    """fp32 (scalar kernels): the first tokens of the sequence masked, no initial state."""
    from causal_flare import flare_autoregressive_prefill_triton
    _print_case("masked_prefill_fp32")
    B, T, H, M, D = 2, 300, 2, 64, 32
    q, k, v = seeded(5, B, T, H, M, D, D, torch.float32)
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[:, :70] = 0
    mask[1, 150:160] = 0
    y, st = flare_autoregressive_prefill_triton(q.to(DEV), k.to(DEV), v.to(DEV), attention_mask=mask.to(DEV))
    y_ref, st_ref = O.ar_recurrent(q, k, v, attention_mask=mask, nthreads=16)
    assert_parity(y, y_ref, torch.float32, "masked prefill fp32")
    assert_state_parity(st, st_ref, torch.float32, "masked prefill fp32")


def test_cfg4_decode_bf16():
    """B=64, H=16, M=128, D=64, 2048-token prefill, then all 256
    decode steps, each output and the final in-place fp32 state against the oracle."""
    from causal_flare import flare_autoregressive_decode_triton, flare_autoregressive_prefill_triton
    _print_case("cfg4")
    B, T, H, M, D, steps = 64, 2048, 16, 128, 64, 256
    torch.manual_seed(3)
    q = (torch.randn(H, M, D) / math.sqrt(D)).to(torch.bfloat16)
    k = torch.randn(B, T + steps, H, D).to(torch.bfloat16)
    v = torch.randn(B, T + steps, H, D).to(torch.bfloat16)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    y, st = flare_autoregressive_prefill_triton(qg, kg[:, :T], vg[:, :T])
    u0 = st["u"]
    ys = []
    for t in range(T, T + steps):
        y_t, st = flare_autoregressive_decode_triton(qg, kg[:, t], vg[:, t], state=st)
        ys.append(y_t)
    assert st["u"] is u0, "decode must update the state in place"
    y_dec = torch.cat(ys, dim=1)
    ref, st_ref = O.ar_recurrent(q, k, v, nthreads=16)
    assert_parity(y, ref[:, :T], torch.bfloat16, "cfg4 prefill")
    assert_parity(y_dec, ref[:, T:], torch.bfloat16, "cfg4 decode (256 steps)")
    assert_state_parity(st, st_ref, torch.bfloat16, "cfg4 after 256 steps")


@pytest.mark.parametrize("M,D,dtype,sep", [(256, 64, torch.bfloat16, False), (256, 64, torch.float16, True),
                                            (64, 128, torch.bfloat16, True), (128, 32, torch.float32, False),
                                            (32, 256, torch.bfloat16, False)])
def test_decode_fast_step_shapes(M, D, dtype, sep):
    """The fast decode step over its template range (rows of u per thread 1..16, 16-byte
    pieces of the Q row above and below the 8 it prefetches, separate decoder tensors):
    a few steps after a prefill, outputs and the in-place state against the oracle (the
    state row-wise: 40 tokens leave single entries of z cancelling to near zero)."""
    from causal_flare import flare_autoregressive_decode_triton, flare_autoregressive_prefill_triton
    _print_case("decode_fast", M, D, dtype, sep)
    B, T, H, steps = 3, 40, 2, 4
    q, k, v = seeded(77 + M + D, B, T + steps, H, M, D, D, dtype, q_std=D ** -0.5)
    g = torch.Generator().manual_seed(78)
    qd = torch.randn((B, T + steps, H, D), generator=g).to(dtype) if sep else None
    kd = (torch.randn((H, M, D), generator=g) * D ** -0.5).to(dtype) if sep else None
    dev = lambda x: None if x is None else x.to(DEV)
    y, st = flare_autoregressive_prefill_triton(dev(q), dev(k[:, :T]), dev(v[:, :T]),
                                                Q_dec=dev(None if qd is None else qd[:, :T]), K_dec=dev(kd))
    ys = []
    for t in range(T, T + steps):
        y_t, st = flare_autoregressive_decode_triton(dev(q), dev(k[:, t]), dev(v[:, t]), state=st,
                                                     Q_dec=dev(None if qd is None else qd[:, t]), K_dec=dev(kd))
        ys.append(y_t)
    ref, st_ref = O.ar_recurrent(q, k, v, Q_dec=qd, K_dec=kd, nthreads=16)
    assert_parity(torch.cat(ys, dim=1), ref[:, T:], dtype, f"decode M={M} D={D} {dtype} sep={sep}")
    assert_state_rowwise((st["m"], st["d"], st["u"]), (st_ref["m"], st_ref["d"], st_ref["u"]), dtype,
                         f"decode state M={M} D={D} {dtype} sep={sep}")


def test_decode_masked_rows_keep_state():
    from causal_flare import flare_autoregressive_decode_triton, flare_autoregressive_prefill_triton
    _print_case("decode_mask")
    B, T, H, M, D = 4, 20, 2, 16, 16
    q, k, v = seeded(21, B, T + 1, H, M, D, D, torch.float32, device=DEV)
    _, st = flare_autoregressive_prefill_triton(q, k[:, :T], v[:, :T])
    before = {kk: vv.clone() for kk, vv in st.items()}
    mask = torch.tensor([1, 0, 1, 0], device=DEV)
    y, st = flare_autoregressive_decode_triton(q, k[:, T], v[:, T], state=st, attention_mask=mask)
    assert float(y[1].abs().max()) == 0.0 and float(y[3].abs().max()) == 0.0
    for kk in ("m", "d", "u"):
        assert torch.equal(st[kk][1], before[kk][1]) and torch.equal(st[kk][3], before[kk][3])
    _, st_o = O.ar_recurrent(q, k[:, :T], v[:, :T])
    y_ref, _ = O.ar_recurrent(q, k[:, T:], v[:, T:], state=st_o, attention_mask=mask.cpu()[:, None])
    assert_parity(y, y_ref, torch.float32, "masked decode")


# --------------------------------------------------------------------------
# Semi-autoregressive (block-causal)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("block_size,chunk_size,seq_len", [(16, 16, 48), (32, 16, 64), (64, 16, 128)])
def test_semi_ar_small_fp32(block_size, chunk_size, seq_len):
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("semi_small", block_size, seq_len)
    B, H, M, D = 2, 3, 5, 16
    q, k, v = seeded(0, B, seq_len, H, M, D, D, torch.float32, device=DEV)
    y, aux = flare_semi_autoregressive_trition(q, k, v, block_size=block_size, chunk_size=chunk_size)
    y_ref, lse_dec, lse_enc = O.semi_ar(q, k, v, block_size, chunk_size)
    assert y.dtype == v.dtype
    assert aux["LSE_dec"].shape == (B, H, seq_len)
    assert aux["LSE_enc"].shape == (B, H, seq_len // block_size, M)
    assert_parity(y, y_ref, torch.float32, "semi y")
    assert_parity(aux["LSE_dec"], lse_dec, torch.float32, "semi LSE_dec")
    assert_parity(aux["LSE_enc"], lse_enc, torch.float32, "semi LSE_enc")


def test_semi_ar_decoder_variants_bf16():
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("semi_variants")
    B, N, H, M, D = 1, 128, 2, 16, 16
    q, k, v = seeded(2, B, N, H, M, D, D, torch.bfloat16, device=DEV)
    g = torch.Generator().manual_seed(4)
    qds, kds = _dec_variants(q, k, g)
    for qn, qd in qds.items():
        for kn, kd in kds.items():
            y, aux = flare_semi_autoregressive_trition(q, k, v, block_size=64, chunk_size=16, Q_dec=qd, K_dec=kd)
            y_ref, _, lse_enc = O.semi_ar(q, k, v, 64, 16, Q_dec=_oracle_dec(qd, k), K_dec=_oracle_dec(kd, q))
            assert_parity(y, y_ref, torch.bfloat16, f"semi q_dec={qn} k_dec={kn}")
            assert_parity(aux["LSE_enc"], lse_enc, torch.bfloat16, "semi LSE_enc")


@pytest.mark.parametrize("M,D,block", [(128, 64, 64), (256, 128, 32)])
@pytest.mark.parametrize("mode", ["sep_q", "sep_k", "both"])
def test_semi_ar_separate_decoder_mfma_bf16(M, D, block, mode):
    """Separate decoder tensors on the block-causal MFMA readout (decoder softmax
    and LSE_dec from the decoder pass)."""
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("semi_sep_mfma", M, D, block, mode)
    B, N, H = 2, 1024, 2
    q, k, v = seeded(61 + M, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    g = torch.Generator().manual_seed(D)
    qd = torch.randn(B, N, H, D, generator=g).bfloat16() if mode in ("sep_q", "both") else None
    kd = (torch.randn(H, M, D, generator=g) * D ** -0.5).bfloat16() if mode in ("sep_k", "both") else None
    dev = lambda t: None if t is None else t.to(DEV)
    y, aux = flare_semi_autoregressive_trition(dev(q), dev(k), dev(v), block_size=block, chunk_size=block,
                                               Q_dec=dev(qd), K_dec=dev(kd))
    y_ref, lse_dec, lse_enc = O.semi_ar(q, k, v, block, block, Q_dec=qd, K_dec=kd)
    assert_parity(y, y_ref, torch.bfloat16, f"semi sep M={M} D={D} {mode}")
    assert_parity(aux["LSE_dec"], lse_dec, torch.bfloat16, "semi sep LSE_dec")
    assert_parity(aux["LSE_enc"], lse_enc, torch.bfloat16, "semi sep LSE_enc")


@pytest.mark.parametrize("M,D,block,N", [(128, 64, 96, 1152), (256, 128, 256, 1024), (128, 128, 512, 1024),
                                         (256, 64, 160, 960), (128, 64, 1024, 1024)])
@pytest.mark.parametrize("mode", ["shared", "both"])
def test_semi_ar_large_blocks_mfma_bf16(M, D, block, N, mode):
    """Blocks whose decoder softmax does not fit in LDS (any multiple of 32 tokens):
    the MFMA readout keeps it in the workspace, written from the shared scores or by
    the decoder pass.  Odd subtile counts (96 = 3 x 32, 160 = 5 x 32) and block = N
    included; chunk_size is only a launch hint in the reference."""
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("semi_large_block", M, D, block, N, mode)
    B, H = 2, 2
    q, k, v = seeded(7 * block + M, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    g = torch.Generator().manual_seed(block)
    qd = torch.randn(B, N, H, D, generator=g).bfloat16() if mode == "both" else None
    kd = (torch.randn(H, M, D, generator=g) * D ** -0.5).bfloat16() if mode == "both" else None
    dev = lambda t: None if t is None else t.to(DEV)
    y, aux = flare_semi_autoregressive_trition(dev(q), dev(k), dev(v), block_size=block, chunk_size=32,
                                               Q_dec=dev(qd), K_dec=dev(kd))
    y_ref, lse_dec, lse_enc = O.semi_ar(q, k, v, block, 32, Q_dec=qd, K_dec=kd, nthreads=16)
    assert_parity(y, y_ref, torch.bfloat16, f"semi large block M={M} D={D} block={block} {mode}")
    if mode == "shared":
        np.testing.assert_allclose(to_np(aux["LSE_dec"]), lse_dec, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(to_np(aux["LSE_enc"]), lse_enc, rtol=1e-4, atol=1e-4)
    else:
        assert_parity(aux["LSE_dec"], lse_dec, torch.bfloat16, "semi large block LSE_dec")
        assert_parity(aux["LSE_enc"], lse_enc, torch.bfloat16, "semi large block LSE_enc")


def test_cfg5_semi_ar_bf16():
    """B=2, N=8192, H=16, M=128, D=64, block 64, bf16, seed 4."""
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("cfg5")
    q, k, v = _cfg_inputs(4, 2, 8192, 16, 128, 64, torch.bfloat16)
    y, aux = flare_semi_autoregressive_trition(q.to(DEV), k.to(DEV), v.to(DEV), block_size=64, chunk_size=64)
    y_ref, lse_dec, _ = O.semi_ar(q, k, v, 64, 64, nthreads=16)
    assert_parity(y, y_ref, torch.bfloat16, "cfg5 y")
    assert_parity(aux["LSE_dec"], lse_dec, torch.bfloat16, "cfg5 LSE_dec")


def test_semi_ar_full_block_equals_noncausal_flare():
    """block_size = N: every token sees every token (semi reference.py:575-596)."""
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("semi_full_block")
    B, N, H, M, D = 2, 64, 2, 16, 32
    q, k, v = seeded(8, B, N, H, M, D, D, torch.float32, device=DEV)
    y, _ = flare_semi_autoregressive_trition(q, k, v, block_size=N, chunk_size=64)
    ref = O.brute_semi_ar(q, k, v, N)
    assert_parity(y, ref, torch.float32, "semi block=N")


# --------------------------------------------------------------------------
# Shapes served by the bf16 MFMA kernels (M in {128, 256}, D in {64, 128})
# --------------------------------------------------------------------------
@pytest.mark.parametrize("M,D", [(128, 64), (128, 128), (256, 64), (256, 128)])
@pytest.mark.parametrize("N,chunk", [(77, None), (1000, 64), (1000, 96), (3000, None)])
def test_mfma_shapes_bf16(M, D, N, chunk):
    from causal_flare import flare_autoregressive_triton
    _print_case("mfma_shapes", M, D, N, chunk)
    B, H = 2, 2
    q, k, v = seeded(31 + M + D, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5, device=DEV)
    y = flare_autoregressive_triton(q, k, v, chunk_size=chunk)
    ref = O.ar_chunked(q, k, v, nthreads=16)
    assert_parity(y, ref, torch.bfloat16, f"mfma M={M} D={D} N={N} chunk={chunk}")


@pytest.mark.parametrize("M,D", [(128, 64), (128, 128), (256, 64), (256, 128)])
@pytest.mark.parametrize("mode", ["sep_q", "sep_k", "both"])
def test_mfma_separate_decoder_bf16(M, D, mode):
    """Separate decoder tensors on the MFMA path: the decoder softmax from its own
    MFMA pass, read by the producer waves (ragged N, several chunks)."""
    from causal_flare import flare_autoregressive_triton
    _print_case("mfma_sep_decoder", M, D, mode)
    B, N, H = 2, 1000, 2
    q, k, v = seeded(41 + M + D, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    g = torch.Generator().manual_seed(M + D)
    qd = torch.randn(B, N, H, D, generator=g).bfloat16() if mode in ("sep_q", "both") else None
    kd = (torch.randn(H, M, D, generator=g) * D ** -0.5).bfloat16() if mode in ("sep_k", "both") else None
    dev = lambda t: None if t is None else t.to(DEV)
    for chunk in (None, 64):
        y = flare_autoregressive_triton(dev(q), dev(k), dev(v), chunk_size=chunk, Q_dec=dev(qd), K_dec=dev(kd))
        ref = O.ar_chunked(q, k, v, Q_dec=qd, K_dec=kd, nthreads=16)
        assert_parity(y, ref, torch.bfloat16, f"mfma sep decoder M={M} D={D} {mode} chunk={chunk}")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
def test_masked_prefill_separate_decoder_bf16(M, D):
    """Masked prefill with separate decoder tensors (MFMA path): masked tokens get
    decoder weights 0 and y = 0, and leave the state unchanged."""
    from causal_flare import flare_autoregressive_prefill_triton
    _print_case("masked_prefill_sep", M, D)
    B, T, H = 2, 700, 2
    q, k, v = seeded(13 + M, B, T, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    g = torch.Generator().manual_seed(3)
    qd = torch.randn(B, T, H, D, generator=g).bfloat16()
    kd = (torch.randn(H, M, D, generator=g) * D ** -0.5).bfloat16()
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[:, :40] = 0
    mask[1, 300:333] = 0
    y, st = flare_autoregressive_prefill_triton(q.to(DEV), k.to(DEV), v.to(DEV), attention_mask=mask.to(DEV),
                                                Q_dec=qd.to(DEV), K_dec=kd.to(DEV))
    y_ref, st_ref = O.ar_recurrent(q, k, v, attention_mask=mask, Q_dec=qd, K_dec=kd, nthreads=16)
    assert torch.all(y[mask == 0].float() == 0), "masked tokens must give y = 0"
    assert_parity(y, y_ref, torch.bfloat16, f"masked prefill sep decoder M={M} D={D}")
    assert_state_parity(st, st_ref, torch.bfloat16, "masked prefill sep decoder")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
def test_mfma_large_values_bf16(M, D):
    """Values far outside fp16 (|v| up to 1e5, also at a chunk start) on the MFMA
    path: the output kernel keeps V and the numerator under a power-of-two scale."""
    from causal_flare import flare_autoregressive_triton
    _print_case("mfma_large_values", M, D)
    B, N, H = 1, 3000, 2
    q, k, v = seeded(57 + M, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    v = v.float()
    v[:, 500:510] *= 1e5      # inside a chunk
    v[:, 1024:1030, 1] *= 3e4  # the start of a chunk (prefix z large for the next ones)
    v = v.bfloat16()
    y = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV), chunk_size=256)
    ref = O.ar_chunked(q, k, v, nthreads=16)
    a, b = to_np(y), np.asarray(ref, np.float64)
    assert np.isfinite(a).all(), "non-finite output with large values"
    # tokens before the first outlier: the ordinary bf16 bar
    assert_parity(y[:, :500], ref[:, :500], torch.bfloat16, f"mfma large values, before M={M} D={D}")
    # after it: fp16 MFMA operands carry ~2^-12 relative error per term, and outputs that
    # cancel terms of size 1e5 keep that error in absolute terms; bound the error by the
    # output scale of each (b, h) sequence
    scale = np.abs(b[:, 500:]).max(axis=(1, 3), keepdims=True)
    err = float((np.abs(a[:, 500:] - b[:, 500:]) / scale).max())
    assert err <= 1e-2, f"mfma large values M={M} D={D}: max |err| / max |ref| = {err:.3e}"


@pytest.mark.parametrize("qk_std", [1.0, 3.0])
def test_mfma_prefill_with_state_bf16(qk_std):
    """Prefill from a cached state on the MFMA path, with larger score spreads."""
    from causal_flare import flare_autoregressive_decode_triton, flare_autoregressive_prefill_triton
    _print_case("mfma_prefill_state", qk_std)
    B, T, H, M, D = 2, 700, 2, 128, 64
    q, k, v = seeded(77, B, 2 * T, H, M, D, D, torch.bfloat16, q_std=qk_std * D ** -0.5, device=DEV)
    scale = 1.0
    _, st = flare_autoregressive_prefill_triton(q, k[:, :T], v[:, :T], scale=scale)
    y, st2 = flare_autoregressive_prefill_triton(q, k[:, T:], v[:, T:], state=st, scale=scale)
    y_ref, st_ref = O.ar_recurrent(q, k, v, scale=scale, nthreads=16)
    if qk_std <= 1.0:
        assert_parity(y, y_ref[:, T:], torch.bfloat16, "mfma prefill with state")
        assert_state_parity(st2, st_ref, torch.bfloat16, "mfma prefill")
    else:   # sharp softmax: bf16 rounding dominates; the reference suite's noise-model policy
        assert_noise_model(y, y_ref[:, T:], "mfma prefill with state (sharp)")
        z = to_np(st2["u"]) / to_np(st2["d"])[..., None]
        assert_noise_model(z, st_ref["u"] / st_ref["d"][..., None], "mfma prefill state z (sharp)")
    y1, _ = flare_autoregressive_decode_triton(q, k[:, -1], v[:, -1], state=st2, scale=scale)
    assert torch.isfinite(y1.float()).all()


@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("qk_std", [0.5, 1.0, 2.0, 4.0])
@pytest.mark.parametrize("dec_mode", ["shared", "sep_q", "sep_k"])
def test_reference_correctness_suite_bf16(D, qk_std, dec_mode):
    """The reference's bf16 correctness sweep (testing/suite_runners/correctness.py:33-113):
    B=1, H=2, N=1024, M=128, q,k ~ qk_std N(0,1), scale D^-0.5, against the
    fp64 two-SDPA definition.  D=64 runs the MFMA kernels (shared decoder)."""
    from causal_flare import flare_autoregressive_triton
    _print_case("ref_suite", D, qk_std, dec_mode)
    B, H, N, M = 1, 2, 1024, 128
    g = torch.Generator().manual_seed(int(100 * qk_std) + D)
    q = (qk_std * torch.randn(H, M, D, generator=g)).bfloat16()
    k = (qk_std * torch.randn(B, N, H, D, generator=g)).bfloat16()
    v = torch.randn(B, N, H, D, generator=g).bfloat16()
    qd = (qk_std * torch.randn(B, N, H, D, generator=g)).bfloat16() if dec_mode == "sep_q" else None
    kd = (qk_std * torch.randn(H, M, D, generator=g)).bfloat16() if dec_mode == "sep_k" else None
    y = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV), scale=D ** -0.5,
                                    Q_dec=None if qd is None else qd.to(DEV), K_dec=None if kd is None else kd.to(DEV))
    ref = O.brute_ar(q, k, v, scale=D ** -0.5, Q_dec=qd, K_dec=kd)
    assert_noise_model(y, ref, f"suite D={D} qk={qk_std} {dec_mode}")
    if qk_std <= 1.0:
        assert_parity(y, ref, torch.bfloat16, f"suite D={D} qk={qk_std} {dec_mode}")


@pytest.mark.parametrize("M,D", [(128, 64), (128, 128), (256, 64), (256, 128)])
@pytest.mark.parametrize("block", [32, 64, 128])
def test_semi_ar_mfma_shapes_bf16(M, D, block):
    """Shapes served by the block-causal MFMA readout (M = 256 with block 128 keeps
    the decoder softmax in the workspace instead of LDS)."""
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("semi_mfma", M, D, block)
    B, N, H = 2, 1024, 2
    q, k, v = seeded(91 + M + D + block, B, N, H, M, D, D, torch.bfloat16, q_std=D ** -0.5, device=DEV)
    y, aux = flare_semi_autoregressive_trition(q, k, v, block_size=block, chunk_size=32)
    y_ref, lse_dec, lse_enc = O.semi_ar(q, k, v, block, 32, nthreads=16)
    assert y.dtype == torch.bfloat16
    assert_parity(y, y_ref, torch.bfloat16, f"semi mfma M={M} D={D} block={block}")
    np.testing.assert_allclose(to_np(aux["LSE_dec"]), lse_dec, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(to_np(aux["LSE_enc"]), lse_enc, rtol=1e-4, atol=1e-4)


# --------------------------------------------------------------------------
# fp16 inputs: the reference computes fp16 inputs in fp16 MMA
# (_get_chunked_forward_config, training.py:315-326) with the 1e-2 bar of
# _get_allclose_tols (_common.py:132-137); here they run on the same
# producer / consumer MFMA kernels as bf16 (fp16 MFMA on the raw input words)
# --------------------------------------------------------------------------
@pytest.mark.parametrize("M,D,N,chunk", [(128, 64, 600, None), (256, 128, 330, None), (128, 128, 300, 64),
                                         (256, 64, 300, 64)])
def test_mfma_fp16_forward(M, D, N, chunk):
    from causal_flare import flare_autoregressive_triton
    _print_case("mfma_fp16", M, D, N, chunk)
    B, H = 2, 2
    q, k, v = seeded(71 + M + D, B, N, H, M, D, D, torch.float16, q_std=D ** -0.5, device=DEV)
    y = flare_autoregressive_triton(q, k, v, chunk_size=chunk)
    assert y.dtype == torch.float16
    ref = O.ar_chunked(q, k, v, nthreads=16)
    assert_parity(y, ref, torch.float16, f"mfma fp16 M={M} D={D} N={N} chunk={chunk}")


@pytest.mark.parametrize("M,D", [(128, 64), (256, 128)])
@pytest.mark.parametrize("mode", ["sep_q", "both"])
def test_mfma_fp16_separate_decoder(M, D, mode):
    from causal_flare import flare_autoregressive_triton
    _print_case("mfma_fp16_sep", M, D, mode)
    B, N, H = 1, 300, 2
    q, k, v = seeded(43 + M + D, B, N, H, M, D, D, torch.float16, q_std=D ** -0.5)
    g = torch.Generator().manual_seed(M + D + 1)
    qd = torch.randn(B, N, H, D, generator=g).half()
    kd = (torch.randn(H, M, D, generator=g) * D ** -0.5).half() if mode == "both" else None
    dev = lambda t: None if t is None else t.to(DEV)
    y = flare_autoregressive_triton(dev(q), dev(k), dev(v), Q_dec=dev(qd), K_dec=dev(kd))
    ref = O.brute_ar(q, k, v, scale=D ** -0.5, Q_dec=qd, K_dec=kd)
    assert_parity(y, ref, torch.float16, f"mfma fp16 sep M={M} D={D} {mode}")


def test_masked_prefill_fp16():
    from causal_flare import flare_autoregressive_prefill_triton
    _print_case("masked_prefill_fp16")
    B, T, H, M, D = 2, 300, 2, 128, 64
    q, k, v = seeded(17, B, T, H, M, D, D, torch.float16, q_std=D ** -0.5)
    mask = torch.ones(B, T, dtype=torch.int64)
    mask[:, :40] = 0
    mask[1, 200:233] = 0
    y, st = flare_autoregressive_prefill_triton(q.to(DEV), k.to(DEV), v.to(DEV), attention_mask=mask.to(DEV))
    y_ref, st_ref = O.ar_recurrent(q, k, v, attention_mask=mask, nthreads=16)
    assert torch.all(y[mask == 0].float() == 0), "masked tokens must give y = 0"
    assert_parity(y, y_ref, torch.float16, "masked prefill fp16")
    assert_state_parity(st, st_ref, torch.float16, "masked prefill fp16")


def test_mfma_fp16_large_values():
    """Values near the fp16 limit: the output kernel's power-of-two V scale keeps the
    numerator finite."""
    from causal_flare import flare_autoregressive_triton
    _print_case("mfma_fp16_large_values")
    B, N, H, M, D = 1, 800, 2, 128, 64
    q, k, v = seeded(59, B, N, H, M, D, D, torch.float16, q_std=D ** -0.5)
    v = v.float()
    v[:, 500:510] = v[:, 500:510].sign() * 6e4
    v = v.half()
    y = flare_autoregressive_triton(q.to(DEV), k.to(DEV), v.to(DEV), chunk_size=256)
    ref = O.ar_chunked(q, k, v, nthreads=16)
    a, b = to_np(y), np.asarray(ref, np.float64)
    assert np.isfinite(a).all(), "non-finite output with large fp16 values"
    assert_parity(y[:, :500], ref[:, :500], torch.float16, "mfma fp16 large values, before")
    scale = np.abs(b[:, 500:]).max(axis=(1, 3), keepdims=True)
    err = float((np.abs(a[:, 500:] - b[:, 500:]) / scale).max())
    assert err <= 1e-2, f"mfma fp16 large values: max |err| / max |ref| = {err:.3e}"


@pytest.mark.parametrize("M,D,block", [(128, 64, 64), (256, 128, 32), (256, 128, 128)])
def test_semi_ar_mfma_fp16(M, D, block):
    from causal_flare import flare_semi_autoregressive_trition
    _print_case("semi_mfma_fp16", M, D, block)
    B, N, H = 1, 512, 2
    q, k, v = seeded(97 + M + D + block, B, N, H, M, D, D, torch.float16, q_std=D ** -0.5, device=DEV)
    y, aux = flare_semi_autoregressive_trition(q, k, v, block_size=block, chunk_size=32)
    assert y.dtype == torch.float16
    y_ref, lse_dec, lse_enc = O.semi_ar(q, k, v, block, 32, nthreads=16)
    assert_parity(y, y_ref, torch.float16, f"semi mfma fp16 M={M} D={D} block={block}")
    np.testing.assert_allclose(to_np(aux["LSE_dec"]), lse_dec, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(to_np(aux["LSE_enc"]), lse_enc, rtol=1e-4, atol=1e-4)


# --------------------------------------------------------------------------
# profile=True: per-phase timings and kernel resources
# --------------------------------------------------------------------------
@pytest.mark.parametrize("M,D,waves", [(128, 64, 4), (256, 128, 8)])
def test_profile_reports_timings_and_kernel_resources(M, D, waves):
    """profile=True returns (Y, dict) with per-phase forward timings and totals
    (reference training.py:4-50) and, per phase, the launched kernel's waves per
    workgroup, VGPRs, spills and LDS bytes (the reference's backward_resources
    record, training.py:4-18, 4418); Y equals the call without profile."""
    from causal_flare import flare_autoregressive_triton
    _print_case("profile_resources", M, D)
    q, k, v = seeded(9, 1, 700, 2, M, D, D, torch.bfloat16, q_std=D ** -0.5)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    y, prof = flare_autoregressive_triton(qd, kd, vd, profile=True)
    assert torch.equal(y, flare_autoregressive_triton(qd, kd, vd))
    assert set(prof["forward"]) == {"flare_chunk_prepare", "flare_chunk_prefix", "flare_chunk_fwd"}
    assert all(t > 0 for t in prof["forward"].values())
    assert prof["total_ms"] == pytest.approx(prof["forward_total_ms"] + prof["backward_total_ms"])
    res = prof["forward_resources"]
    assert set(res) == {"flare_chunk_prepare", "flare_chunk_prefix", "flare_chunk_fwd"}
    for name, r in res.items():
        assert 0 < r["regs_per_thread"] <= 512 and r["spills"] >= 0, (name, r)
    assert res["flare_chunk_prepare"]["num_waves"] == M // 32
    assert res["flare_chunk_fwd"]["num_waves"] == M // 64 + D // 32
    assert res["flare_chunk_fwd"]["shared_bytes"] > 32 * 1024 and res["flare_chunk_prepare"]["shared_bytes"] > 0
    assert waves == M // 32
