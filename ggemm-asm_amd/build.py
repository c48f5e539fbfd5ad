"""In-tree build of the HIP artefacts for gfx950.

* ``lib/libggemm_vark.so`` -- the extern "C" launcher library (include/ggemm_vark.h) with the
  tensorwise, K=32-MFMA and MXFP8 kernels.
* ``lib/variable_k_wgrad.co`` -- the drop-in code object exporting only
  ``_grouped_variable_k_gemm_kernel`` with the reference kernarg layout.
"""
from __future__ import annotations

import os
import shutil
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
SO_PATH = os.path.join(LIB_DIR, "libggemm_vark.so")
CO_PATH = os.path.join(LIB_DIR, "variable_k_wgrad.co")
ARCH = "gfx950"

# Packed-FP32 VALU ops are disabled for all device code (they are left to no hand-written use).
DEVICE_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else (shutil.which("hipcc") or "hipcc")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed ({r.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, flush=True)


def build_so(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = SO_PATH + ".tmp"
    _run([hipcc(), *DEVICE_FLAGS, "-fPIC", "-shared", os.path.join(CSRC, "vark_capi.hip"), "-o", tmp], verbose)
    os.replace(tmp, SO_PATH)
    return SO_PATH


def build_co(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = CO_PATH + ".tmp"
    # a raw AMDGPU ELF (not a clang offload bundle), like the reference's code object
    _run([hipcc(), *DEVICE_FLAGS, "--cuda-device-only", "--no-gpu-bundle-output",
          os.path.join(CSRC, "vark_co.hip"), "-o", tmp], verbose)
    os.replace(tmp, CO_PATH)
    return CO_PATH


def build_all(verbose: bool = False) -> tuple[str, str]:
    return build_so(verbose), build_co(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
