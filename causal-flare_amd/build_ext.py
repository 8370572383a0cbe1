"""Build the HIP library ``causal_flare/_lib/libflare_mi355x.so`` for gfx950.

Every ``csrc/*.hip`` / ``csrc/*.cpp`` file is compiled with ``hipcc`` into an
object file and linked into one shared library.  The library links against the
HIP runtime that PyTorch itself loads (``torch/lib/libamdhip64.so``) so that one
process never holds two HIP runtimes; the rpath points there.

Usage: ``python causal-flare_amd/build_ext.py`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "causal_flare", "_lib")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libflare_mi355x.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled: the compiler must not form v_pk_*_f32.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-munsafe-fp-atomics",
]

# Per-file additions.  chunk_prepare_tr: MFMA accumulators in VGPRs rather than AGPRs, so
# that the exponentials read the scores (and the rare rescale reads U) without a
# v_accvgpr_read per value each tile (measured: config 2 prepare 25.9 -> 23.8 us); the
# backward's per-chunk kernels (config 3 backward 21.5 -> 20.9 ms) and the decoder softmax
# pass of separate decoder tensors (config-2 shape forward 0.127 -> 0.121 ms) likewise.
FILE_FLAGS = {
    "flare_ar_prep.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "flare_ar_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "flare_ar_pc.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _torch_lib_dir() -> str:
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        raise RuntimeError("torch is required to locate the HIP runtime it ships")
    return os.path.join(list(spec.submodule_search_locations)[0], "lib")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), *lang, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    warn = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l and "not a recognized feature" not in l)
    if warn.strip():
        print(warn, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tlib = _torch_lib_dir()
    out = os.path.join(OUT_DIR, LIB_NAME)
    tmp = out + ".tmp"
    # Link through the host compiler: hipcc would add /opt/rocm's own runtime.
    cmd = ["g++", "-shared", "-fPIC", *objs, "-o", tmp, f"-L{tlib}", "-l:libamdhip64.so",
           f"-Wl,-rpath,{tlib}", "-Wl,--no-undefined"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build()
