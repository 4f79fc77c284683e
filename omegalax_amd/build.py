"""Build libomx_gdn.so for gfx950 with hipcc (in-tree, no JIT cache).

    python -m omegalax_amd.build          # compile every source, link the library

Sources are omegalax_amd/csrc/*.hip (device code) and *.cpp (the C ABI); objects go
to omegalax_amd/_build/ and the library to omegalax_amd/lib/libomx_gdn.so.  When JAX is
installed, the XLA FFI handlers (omegalax_amd/xla/gdn_xla_ffi.cc) are built as well, into
omegalax_amd/lib/libomx_gdn_xla.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libomx_gdn.so")
ROOT = os.path.dirname(PKG)

ARCH = "gfx950"
# Packed fp32 VALU ops are disabled: some of their forms have given silently wrong
# results on these boxes, so the compiler must not form them from float code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-Wall",
          "-Wno-unused-function", "-I", os.path.join(ROOT, "include"), "-I", CSRC]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libomx_gdn.so)")


# MFMA-heavy sources: keep MFMA accumulators in VGPRs, so the VALU work on them
# (scaling, packing to bf16) needs no AGPR<->VGPR copies
MFMA_VGPR_SOURCES = {"gdn_chunk.hip", "gdn_prep.hip", "gdn_qkv.hip"}
MFMA_VGPR_FLAGS = ["-mllvm", "-amdgpu-mfma-vgpr-form"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    extra = MFMA_VGPR_FLAGS if os.path.basename(src) in MFMA_VGPR_SOURCES else []
    cmd = [hipcc(), *COMMON, *DEVICE_FLAGS, *extra, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [hipcc(), *COMMON, "-x", "hip", *DEVICE_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that is harmless
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


XLA_SRC = os.path.join(PKG, "xla", "gdn_xla_ffi.cc")
XLA_LIB = os.path.join(LIBDIR, "libomx_gdn_xla.so")


def xla_include_dir():
    """jaxlib's FFI header directory, or None when JAX is not installed."""
    try:
        import jax.ffi
    except ImportError:
        return None
    return jax.ffi.include_dir()


def build_xla_ffi(verbose: bool = True):
    """The optional XLA FFI handlers (omegalax_amd/xla/gdn_xla_ffi.cc), linked against
    libomx_gdn.so; built only when jaxlib's FFI headers are importable."""
    inc = xla_include_dir()
    if inc is None:
        if verbose:
            print("skipped the XLA FFI handlers: jax is not installed")
        return None
    cmd = [hipcc(), *COMMON, "-x", "hip", *DEVICE_FLAGS, "-I", inc, "-shared", XLA_SRC, "-o",
           XLA_LIB, "-L", LIBDIR, "-lomx_gdn", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"XLA FFI build failed: {' '.join(cmd)}\n{r.stderr}")
    if verbose:
        print(f"built {XLA_LIB}")
    return XLA_LIB


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    build_xla_ffi(verbose)
    return LIB


if __name__ == "__main__":
    build()
