"""The allocation-free forward flare_ar_forward_noalloc (static device scratch)
against flare_ar_forward with a caller workspace, through the C ABI: two calls in
a row on one device, the second with a smaller input, each bit-identical to the
workspace entry point; calls on two streams without a host synchronisation in
between (the entry point orders them); plus the size limit."""
import ctypes
import math
import sys

import pytest
import torch

from causal_flare import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _fn():
    lib = _lib.lib()
    return lib, lib.flare_ar_forward_noalloc


def _inputs(seed, B, N, H, M, D, dtype, sep):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(H, M, D, generator=g) / math.sqrt(D)).to(dtype)
    k = torch.randn(B, N, H, D, generator=g).to(dtype)
    v = torch.randn(B, N, H, D, generator=g).to(dtype)
    qd = torch.randn(B, N, H, D, generator=g).to(dtype) if sep else None
    return [None if t is None else t.to(DEV) for t in (q, k, v, qd)]


def _pair(lib, fn, case, seed, B, N, H, M, D, dtype, sep=False, state=False, masked=False):
    print("CASE no_alloc", case, B, N, H, M, D, dtype, sep, state, masked, flush=True)
    sys.stdout.flush()
    q, k, v, qd = _inputs(seed, B, N, H, M, D, dtype, sep)
    code = _lib.dtype_code(dtype)
    scale = D ** -0.5
    st = [None] * 3
    if state:
        st = [torch.randn(B, H, M, device=DEV), torch.rand(B, H, M, device=DEV) + 0.5,
              torch.randn(B, H, M, D, device=DEV)]
    mask = None
    if masked:
        mask = torch.ones(B, N, dtype=torch.int32, device=DEV)
        mask[:, 5:40] = 0
    P = _lib.ptr
    outs = []
    for which in ("ws", "noalloc"):
        y = torch.full((B, N, H, D), float("nan"), device=DEV, dtype=dtype)
        fin = [torch.empty(B, H, M, device=DEV), torch.empty(B, H, M, device=DEV), torch.empty(B, H, M, D, device=DEV)]
        stream = _lib.stream_of(torch.device(DEV))
        if which == "ws":
            size_fn = lib.flare_ar_forward_workspace_size_sep if sep else lib.flare_ar_forward_workspace_size
            nb = size_fn(B, N, H, M, D, 0)
            ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
            rc = lib.flare_ar_forward_masked(P(q), P(k), P(v), P(qd), None, code, B, N, H, M, D, D, scale, 0,
                                             *[P(t) for t in st], *[P(t) for t in fin], P(y), code, P(mask),
                                             P(ws), nb, stream)
        else:
            rc = fn(P(q), P(k), P(v), P(qd), None, code, B, N, H, M, D, D, scale, 0, *[P(t) for t in st],
                    *[P(t) for t in fin], P(y), code, P(mask), stream)
        _lib.check(rc, which)
        torch.cuda.synchronize()
        outs.append((y, fin))
    (y0, f0), (y1, f1) = outs
    assert torch.isfinite(y1.float()).all()
    assert torch.equal(y0, y1), f"{case}: noalloc output differs from the workspace entry point"
    for a, b in zip(f0, f1):
        assert torch.equal(a, b), f"{case}: final state differs"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(dtype):
    lib, fn = _fn()
    # a large call, then a smaller one on the same scratch (its stale contents must not leak in)
    _pair(lib, fn, "large", 1, 2, 4096, 8, 128, 64, dtype)
    _pair(lib, fn, "small", 2, 1, 700, 2, 128, 64, dtype, state=True)
    _pair(lib, fn, "masked", 3, 2, 300, 2, 64, 32, dtype, masked=True)


def test_noalloc_separate_decoder_and_limit():
    lib, fn = _fn()
    _pair(lib, fn, "sep", 4, 2, 1000, 2, 128, 64, torch.bfloat16, sep=True)
    _pair(lib, fn, "sep-small", 5, 1, 200, 2, 128, 64, torch.bfloat16, sep=True)
    # beyond the scratch maximum: a clear error, nothing launched
    cap = lib.flare_ar_forward_noalloc_max_bytes()
    assert cap == 64 << 20
    q, k, v, _ = _inputs(6, 1, 64, 1, 32, 32, torch.bfloat16, False)
    y = torch.empty_like(v)
    rc = fn(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), None, None, _lib.BF16, 64, 1 << 20, 64, 256, 128, 128, 0.1, 64,
            None, None, None, None, None, None, _lib.ptr(y), _lib.BF16, None, _lib.stream_of(torch.device(DEV)))
    assert rc == -1 and b"maximum is" in lib.flare_last_error()


def test_noalloc_calls_on_two_streams_are_ordered():
    """Back-to-back calls on one stream, then on a second stream with no host
    synchronisation in between: the entry point makes the second stream wait for
    the first call's kernels, so both outputs equal the workspace entry point's."""
    lib, fn = _fn()
    P = _lib.ptr
    print("CASE no_alloc two streams", flush=True)
    shapes = [(11, 1, 8192, 8, 128, 64), (12, 2, 2048, 4, 128, 64), (13, 1, 4096, 8, 128, 64)]
    ins, refs = [], []
    for seed, B, N, H, M, D in shapes:
        q, k, v, _ = _inputs(seed, B, N, H, M, D, torch.bfloat16, False)
        nb = lib.flare_ar_forward_workspace_size(B, N, H, M, D, 0)
        ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
        y = torch.empty_like(v)
        _lib.check(lib.flare_ar_forward(P(q), P(k), P(v), None, None, _lib.BF16, B, N, H, M, D, D, D ** -0.5, 0,
                                        None, None, None, None, None, None, P(y), _lib.BF16, P(ws), nb,
                                        _lib.stream_of(torch.device(DEV))), "ws")
        ins.append((q, k, v, B, N, H, M, D))
        refs.append(y)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.full_like(r, float("nan")) for r in refs]
    torch.cuda.synchronize()
    for (q, k, v, B, N, H, M, D), y, s in zip(ins, outs, (s1, s1, s2)):
        rc = fn(P(q), P(k), P(v), None, None, _lib.BF16, B, N, H, M, D, D, D ** -0.5, 0, None, None, None,
                None, None, None, P(y), _lib.BF16, None, ctypes.c_void_p(s.cuda_stream))
        _lib.check(rc, "noalloc")
    torch.cuda.synchronize()
    for i, (y, r) in enumerate(zip(outs, refs)):
        assert torch.equal(y, r), f"call {i}: noalloc output differs from the workspace entry point"
