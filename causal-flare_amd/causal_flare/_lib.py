"""ctypes binding of the HIP library ``_lib/libflare_mi355x.so`` (C ABI in include/flare_mi355x.h).

The library is the only compute path: there is no CPU or eager-PyTorch
fallback.  Importing works without the library (so validation errors can be
raised on a machine without a GPU), but the first call that needs a kernel
raises ``RuntimeError`` if the library is missing or fails to load.
"""
from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# FLARE_LIB_PATH names another build of the same library (A/B comparisons of kernel variants).
LIB_PATH = os.environ.get("FLARE_LIB_PATH") or os.path.join(_HERE, "_lib", "libflare_mi355x.so")
HEADER_FUNCTIONS = (
    "flare_abi_version",
    "flare_last_error",
    "flare_chunk_prepare",
    "flare_chunk_prefix",
    "flare_chunk_output",
    "flare_ar_forward_workspace_size",
    "flare_ar_forward_workspace_size_sep",
    "flare_ar_forward",
    "flare_ar_forward_masked",
    "flare_ar_default_chunk",
    "flare_stablemax_forward",
    "flare_stablemax_backward_workspace_size",
    "flare_stablemax_backward",
    "flare_forward_kernel_resources",
    "flare_ar_backward_workspace_size",
    "flare_ar_backward",
    "flare_decode_step",
    "flare_semi_ar_workspace_size",
    "flare_semi_ar_workspace_size_sep",
    "flare_semi_ar_forward",
    "flare_semi_ar_forward_state",
    "flare_semi_ar_backward_workspace_size",
    "flare_semi_ar_backward",
    "flare_ar_forward_noalloc_max_bytes",
    "flare_ar_forward_noalloc",
    "flare_device_faults",
    "flare_set_meet_spin_limit",
)

F32, BF16, F16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_lib = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t


def _declare(lib):
    lib.flare_abi_version.restype = _i
    lib.flare_abi_version.argtypes = []
    lib.flare_last_error.restype = ctypes.c_char_p
    lib.flare_last_error.argtypes = []
    lib.flare_chunk_prepare.restype = _i
    lib.flare_chunk_prepare.argtypes = [_vp, _vp, _vp, _i] + [_i64] * 6 + [_f, _i64] + [_vp] * 3 + [_vp]
    lib.flare_chunk_prefix.restype = _i
    lib.flare_chunk_prefix.argtypes = [_vp] * 3 + [_i64] * 4 + [_vp] * 6 + [_vp]
    lib.flare_chunk_output.restype = _i
    lib.flare_chunk_output.argtypes = [_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64] + [_vp] * 3 + [_vp, _i, _vp, _vp]
    lib.flare_ar_forward_workspace_size.restype = _sz
    lib.flare_ar_forward_workspace_size.argtypes = [_i64] * 6
    lib.flare_ar_forward_workspace_size_sep.restype = _sz
    lib.flare_ar_forward_workspace_size_sep.argtypes = [_i64] * 6
    lib.flare_ar_default_chunk.restype = _i64
    lib.flare_ar_default_chunk.argtypes = [_i64] * 5
    lib.flare_stablemax_forward.restype = _i
    lib.flare_stablemax_forward.argtypes = [_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64, _f, _vp, _i, _vp, _sz, _vp]
    lib.flare_stablemax_backward_workspace_size.restype = _sz
    lib.flare_stablemax_backward_workspace_size.argtypes = [_i64] * 6 + [_i]
    lib.flare_stablemax_backward.restype = _i
    lib.flare_stablemax_backward.argtypes = [_vp] * 5 + [_i] + [_i64] * 6 + [_f, _f] + [_vp] * 7 + [_vp, _sz, _vp]
    lib.flare_forward_kernel_resources.restype = _i
    lib.flare_forward_kernel_resources.argtypes = [_i] + [_i64] * 3 + [_i, _i64, _i, _vp]
    lib.flare_ar_forward_masked.restype = _i
    lib.flare_ar_forward_masked.argtypes = ([_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64] + [_vp] * 6
                                            + [_vp, _i, _vp, _vp, _sz, _vp])
    lib.flare_ar_forward.restype = _i
    lib.flare_ar_forward.argtypes = ([_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64] + [_vp] * 6
                                     + [_vp, _i, _vp, _sz, _vp])
    lib.flare_ar_backward_workspace_size.restype = _sz
    lib.flare_ar_backward_workspace_size.argtypes = [_i64] * 6
    lib.flare_ar_backward.restype = _i
    lib.flare_ar_backward.argtypes = ([_vp] * 5 + [_i] + [_i64] * 6 + [_f] + [_vp] * 7 + [_vp, _sz, _vp])
    lib.flare_decode_step.restype = _i
    lib.flare_decode_step.argtypes = [_vp] * 6 + [_i] + [_i64] * 5 + [_f] + [_vp] * 3 + [_vp, _i, _vp]
    lib.flare_semi_ar_workspace_size.restype = _sz
    lib.flare_semi_ar_workspace_size.argtypes = [_i64] * 6
    lib.flare_semi_ar_workspace_size_sep.restype = _sz
    lib.flare_semi_ar_workspace_size_sep.argtypes = [_i64] * 6
    lib.flare_semi_ar_backward_workspace_size.restype = _sz
    lib.flare_semi_ar_backward_workspace_size.argtypes = [_i64] * 7
    lib.flare_semi_ar_backward.restype = _i
    lib.flare_semi_ar_backward.argtypes = ([_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64] + [_vp] * 7 + [_vp, _sz, _vp])
    lib.flare_ar_forward_noalloc_max_bytes.restype = _sz
    lib.flare_ar_forward_noalloc_max_bytes.argtypes = []
    lib.flare_ar_forward_noalloc.restype = _i
    lib.flare_ar_forward_noalloc.argtypes = ([_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64] + [_vp] * 6
                                             + [_vp, _i, _vp, _vp])
    lib.flare_device_faults.restype = _i
    lib.flare_device_faults.argtypes = [_vp, ctypes.POINTER(ctypes.c_uint32), _i]
    lib.flare_set_meet_spin_limit.restype = _i
    lib.flare_set_meet_spin_limit.argtypes = [_i]
    lib.flare_semi_ar_forward_state.restype = _i
    lib.flare_semi_ar_forward_state.argtypes = ([_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64] + [_vp] * 6
                                                + [_vp, _i, _vp, _sz, _vp])
    lib.flare_semi_ar_forward.restype = _i
    lib.flare_semi_ar_forward.argtypes = ([_vp] * 5 + [_i] + [_i64] * 6 + [_f, _i64] + [_vp, _i, _vp, _vp]
                                          + [_vp, _sz, _vp])


def _check_single_hip_runtime():
    """Refuse to run with two HIP runtimes mapped (torch's and another)."""
    try:
        with open("/proc/self/maps") as fh:
            paths = {line.split()[-1] for line in fh if "libamdhip64" in line}
    except OSError:
        return
    real = {os.path.realpath(p) for p in paths}
    if len(real) > 1:
        raise RuntimeError(f"two HIP runtimes are loaded in this process: {sorted(real)}")


def lib():
    """Load (once) and return the HIP library; raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"causal_flare HIP library not built: {LIB_PATH} is missing. "
                "Run `python causal-flare_amd/build_ext.py` (or __graft_entry__.build())."
            )
        h = ctypes.CDLL(LIB_PATH)
        _declare(h)
        _check_single_hip_runtime()
        _lib = h
    return _lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16") from None


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def check(rc: int, what: str):
    if rc != 0:
        msg = lib().flare_last_error().decode(errors="replace")
        if rc == -1:
            raise ValueError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def device_faults(device=None, reset: bool = False) -> int:
    """Synchronise the current stream and return the device's count of bounded
    waits that gave up in the output kernel (0 in a healthy run)."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    n = ctypes.c_uint32(0)
    check(lib().flare_device_faults(stream_of(dev), ctypes.byref(n), 1 if reset else 0), "device_faults")
    return int(n.value)


def set_meet_spin_limit(limit: int) -> None:
    """Sleeps before a producer meeting of the output kernel gives up (default 1 << 20)."""
    check(lib().flare_set_meet_spin_limit(int(limit)), "set_meet_spin_limit")
