"""Host-side behaviour that needs no GPU: validation and error messages of the
drop-in entry points, stubs, scale defaults, and that the C-ABI library loads
and exports every function include/flare_mi355x.h declares.

Error cases mirror the reference's CPU tests:
testing/semi_autoregressive/test_block_causal.py:18-41, 260-275 and
testing/autoregressive/test_flare.py:493-518.
"""
import ctypes
import os
import re

import pytest
import torch

import causal_flare
from causal_flare import _lib
from causal_flare._common import _get_allclose_tols, _resolve_attn_scale
from causal_flare._reference_utils import resolve_flare_causal_decode_inputs, validate_flare_qkv_layouts

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flare_mi355x.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(flare_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    declared = _declared_functions()
    assert len(declared) >= 10
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, f"declared in flare_mi355x.h but not exported: {missing}"
    assert set(declared) == set(_lib.HEADER_FUNCTIONS)


def test_library_version_and_host_only_calls():
    lib = _lib.lib()
    assert lib.flare_abi_version() == 1
    assert lib.flare_ar_default_chunk(1, 65536, 16, 256, 128) % 64 == 0
    assert lib.flare_ar_forward_workspace_size(1, 100, 2, 16, 16, 64) >= 4 * (2 * 2 * 2 * 16 + 2 * 2 * 16 * 16)
    # argument validation happens on the host, before any device work
    rc = lib.flare_decode_step(None, None, None, None, None, None, 1, 1, 1, 16, 16, 16, 1.0, None, None, None,
                               None, 1, None)
    assert rc == -1 and b"null pointer" in lib.flare_last_error()
    rc = lib.flare_semi_ar_forward(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, 1,
                                   1, 40, 1, 16, 16, 16, 1.0, 16, ctypes.c_void_p(16), 1, None, None, None, 0,
                                   None)
    assert rc == -1 and b"N % block == 0" in lib.flare_last_error()


def test_public_names_match_reference_exports():
    for name in ("flare_autoregressive_triton", "flare_autoregressive_decode_triton",
                 "flare_autoregressive_prefill_triton", "flare_recurrent_triton",
                 "flare_semi_autoregressive_decode_trition", "flare_semi_autoregressive_prefill_trition",
                 "flare_semi_autoregressive_trition", "autoregressive", "semi_autoregressive"):
        assert hasattr(causal_flare, name), name


@pytest.mark.parametrize(
    ("block_size", "chunk_size", "message"),
    [(24, 16, "multiple of 16"), (32, 48, "currently supports chunk_size"),
     (48, 32, "sequence length N to be an exact multiple of block_size")],
)
def test_semi_ar_validation_messages(block_size, chunk_size, message):
    q = torch.randn((2, 4, 16))
    k = torch.randn((1, 8, 2, 16))
    v = torch.randn((1, 8, 2, 16))
    with pytest.raises(ValueError, match=message):
        causal_flare.flare_semi_autoregressive_trition(q, k, v, block_size=block_size, chunk_size=chunk_size)


def test_semi_ar_rejects_non_block_aligned_length_and_missing_args():
    q = torch.randn((2, 4, 16))
    k = torch.randn((1, 33, 2, 16))
    v = torch.randn((1, 33, 2, 16))
    with pytest.raises(ValueError, match="exact multiple of block_size"):
        causal_flare.flare_semi_autoregressive_trition(q, k, v, block_size=16, chunk_size=16)
    with pytest.raises(ValueError, match="block_size to be specified explicitly"):
        causal_flare.flare_semi_autoregressive_trition(q, k, v, block_size=None, chunk_size=16)
    with pytest.raises(ValueError, match="integer multiple of chunk_size"):
        causal_flare.flare_semi_autoregressive_trition(q, k[:, :32], v[:, :32], block_size=32, chunk_size=64)
    with pytest.raises(ValueError, match="requires CUDA tensors"):
        causal_flare.flare_semi_autoregressive_trition(q, k[:, :32], v[:, :32], block_size=16, chunk_size=16)


def test_semi_ar_cached_validation():
    """The semi-AR cached prefill / block decode (stubs in the reference,
    semi_autoregressive/inference.py:5-36) validate blocks before they need a GPU."""
    q, k, v = torch.randn(2, 4, 16), torch.randn(1, 48, 2, 16), torch.randn(1, 48, 2, 16)
    # block_size is required for a prefill (no whole-call default block)
    with pytest.raises(ValueError, match="requires block_size"):
        causal_flare.flare_semi_autoregressive_prefill_trition(q, k, v)
    with pytest.raises(ValueError, match="requires block_size"):
        causal_flare.semi_autoregressive.SemiAutoRegressivePrefillFLARE.apply(q, k, v)
    with pytest.raises(ValueError, match="multiple of 16"):
        causal_flare.flare_semi_autoregressive_prefill_trition(q, k, v, block_size=24)
    with pytest.raises(ValueError, match="exact multiple of block_size"):
        causal_flare.flare_semi_autoregressive_prefill_trition(q, k, v, block_size=32)
    with pytest.raises(ValueError, match="multiple of 16"):
        causal_flare.flare_semi_autoregressive_decode_trition(q, k[:, :24], v[:, :24])
    with pytest.raises(RuntimeError, match="requires CUDA tensors"):
        causal_flare.flare_semi_autoregressive_prefill_trition(q, k, v, block_size=16)
    with pytest.raises(NotImplementedError, match="attention_mask"):
        causal_flare.flare_semi_autoregressive_prefill_trition(q, k, v, attention_mask=torch.zeros(1, 48))


def test_recurrent_validation_messages():
    """flare_recurrent_triton validates as RecurrentFLARE.forward and the tile helpers
    (recurrent.py:60-116, 291-312) before it needs a GPU."""
    q, k, v = torch.randn(2, 16, 16), torch.randn(1, 8, 2, 16), torch.randn(1, 8, 2, 16)
    with pytest.raises(ValueError, match="Recurrent FLARE expects Q"):
        causal_flare.flare_recurrent_triton(q[0], k, v)
    with pytest.raises(ValueError, match="K and V must have the same shape"):
        causal_flare.flare_recurrent_triton(q, k, torch.randn(1, 8, 2, 32))
    with pytest.raises(ValueError, match="matching H,D"):
        causal_flare.flare_recurrent_triton(torch.randn(3, 16, 16), k, v)
    with pytest.raises(ValueError, match="multiples of 16"):
        causal_flare.flare_recurrent_triton(torch.randn(2, 8, 16), k, v)
    with pytest.raises(ValueError, match="BLOCK_T must be 1 or a multiple of 16"):
        causal_flare.flare_recurrent_triton(q, k, v, block_t=8)
    with pytest.raises(ValueError, match="BLOCK_T currently supports"):
        causal_flare.flare_recurrent_triton(q, k, v, block_t=48)
    with pytest.raises(ValueError, match="BLOCK_M must be a multiple of 16"):
        causal_flare.flare_recurrent_triton(q, k, v, block_m=8)
    with pytest.raises(ValueError, match="BLOCK_D must be a multiple of 16"):
        causal_flare.flare_recurrent_triton(q, k, v, block_d=8)
    with pytest.raises(RuntimeError, match="GPU"):
        causal_flare.flare_recurrent_triton(q, k, v)


def test_autoregressive_shape_assertions_and_cpu_rejection():
    q = torch.randn(2, 16, 16)
    k = torch.randn(1, 8, 2, 16)
    with pytest.raises(AssertionError):
        causal_flare.flare_autoregressive_triton(q, k, torch.randn(1, 9, 2, 16))
    with pytest.raises(AssertionError, match="M must be divisible by 16"):
        causal_flare.flare_autoregressive_triton(torch.randn(2, 12, 16), k, k)
    with pytest.raises(AssertionError, match="CHUNK_SIZE must be divisible by 16"):
        causal_flare.flare_autoregressive_triton(q.cuda() if torch.cuda.is_available() else q, k, k, chunk_size=24)
    with pytest.raises(RuntimeError, match="requires GPU tensors"):
        causal_flare.flare_autoregressive_triton(q, k, k)
    with pytest.raises(RuntimeError, match="requires CUDA tensors"):
        causal_flare.flare_autoregressive_prefill_triton(q, k, k)
    with pytest.raises(RuntimeError, match="requires CUDA tensors"):
        causal_flare.flare_autoregressive_decode_triton(q, k[:, 0], k[:, 0])


def test_decoder_input_validation_messages():
    q = torch.randn(2, 16, 64)
    k = torch.randn(1, 4, 2, 64)
    with pytest.raises(ValueError, match="K_dec and Q_enc must have the same shape"):
        resolve_flare_causal_decode_inputs(q, k, None, torch.randn(2, 16, 80))
    with pytest.raises(ValueError, match="Q_dec and K_enc must have the same shape"):
        resolve_flare_causal_decode_inputs(q, k, torch.randn(1, 4, 2, 80), None)
    with pytest.raises(ValueError, match="Expected Q_dec"):
        resolve_flare_causal_decode_inputs(q, k, torch.randn(4, 2, 64), None)
    qd, kd, sq, sk, shared = resolve_flare_causal_decode_inputs(q, k, k, q)
    assert shared and sq and sk and qd is k and kd is q
    _, _, _, _, shared = resolve_flare_causal_decode_inputs(q, k, None, torch.randn(2, 16, 64))
    assert not shared
    with pytest.raises(ValueError, match="expects Q"):
        validate_flare_qkv_layouts(torch.randn(2, 16), k, k, name="X")


def test_decode_q_dec_shape_validation_message():
    from causal_flare.autoregressive.inference import _canonicalize_q_dec_for_decode
    k_step = torch.randn(1, 2, 64)
    with pytest.raises(ValueError, match="Decode Q_dec"):
        _canonicalize_q_dec_for_decode(torch.randn(1, 1, 2, 80), k_step)
    with pytest.raises(ValueError, match="sequence length 1"):
        _canonicalize_q_dec_for_decode(torch.randn(1, 2, 2, 64), k_step)


def test_state_validation_messages():
    from causal_flare.autoregressive.inference import _canonicalize_flare_state
    with pytest.raises(ValueError, match="must be a dict"):
        _canonicalize_flare_state([1], 1, 2, 16, 16, "cpu")
    with pytest.raises(ValueError, match="Invalid FLARE recurrent state keys"):
        _canonicalize_flare_state({"m": 1}, 1, 2, 16, 16, "cpu")
    bad = {"m": torch.zeros(1, 2, 16), "d": torch.zeros(1, 2, 16), "u": torch.zeros(1, 2, 16, 8)}
    with pytest.raises(ValueError, match="Invalid FLARE recurrent state shapes"):
        _canonicalize_flare_state(bad, 1, 2, 16, 16, "cpu")
    good = {"m": torch.zeros(1, 2, 16), "d": torch.zeros(1, 2, 16), "u": torch.zeros(1, 2, 16, 16)}
    st = _canonicalize_flare_state(good, 1, 2, 16, 16, "cpu")
    assert st["u"] is good["u"], "fp32 state on the right device must be used as is (decode aliasing)"
    fresh = _canonicalize_flare_state(None, 1, 2, 16, 16, "cpu")
    assert torch.isneginf(fresh["m"]).all() and (fresh["d"] == 0).all()


def test_scale_and_tolerance_helpers():
    assert _resolve_attn_scale(None, 8) == 1.0
    assert _resolve_attn_scale(None, 64) == 0.125
    assert _resolve_attn_scale(0.5, 64) == 0.5
    assert _get_allclose_tols(torch.float32) == (1e-5, 1e-5)
    assert _get_allclose_tols(torch.bfloat16) == (1e-2, 1e-2)


def test_input_precision_validation():
    from causal_flare._common import _normalize_input_precision
    assert _normalize_input_precision("tf32x3") == "tf32x3"
    with pytest.raises(ValueError, match="Unsupported input_precision"):
        _normalize_input_precision("fp8")


def test_bench_refuses_multi_gpu():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_stablemax_validation():
    """flare_autoregressive_stablemax_triton keeps the reference's refusals
    (stablemax_triton.py:2441-2452, 1754-1758) and its module export."""
    from causal_flare.autoregressive import flare_autoregressive_stablemax_triton as smx
    from causal_flare.autoregressive import FLAREAutoregressiveStablemaxTriton  # noqa: F401
    q, k, v = torch.randn(2, 16, 16), torch.randn(1, 32, 2, 16), torch.randn(1, 32, 2, 16)
    for kw, msg in ((dict(eps=1e-6), "does not use eps"), (dict(profile=True), "profile=True"),
                    (dict(state={}), "recurrent state"), (dict(attention_mask=torch.ones(1, 32)), "attention_mask"),
                    (dict(return_state=True), "return_state=True"), (dict(write_gate=True), "non-write-gated")):
        with pytest.raises(NotImplementedError, match=re.escape(msg)):
            smx(q, k, v, **kw)
    with pytest.raises(ValueError, match="chunk size divisible by 16"):
        smx(q, k, v, chunk_size=24)
    with pytest.raises(ValueError, match="power must be positive"):
        smx(q, k, v, power=0.0)
    with pytest.raises(RuntimeError, match="requires GPU tensors"):
        smx(q, k, v)
    # N = 0 needs no kernel
    y = smx(q, k[:, :0], v[:, :0])
    assert y.shape == (1, 0, 2, 16) and y.dtype == v.dtype
