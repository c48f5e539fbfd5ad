"""Build recipe for the oracle side (TEST INFRASTRUCTURE ONLY).

* ``oracle/_build/libvark_oracle_c.so`` -- gcc build of the C restatement ``vark_oracle.c``.
* ``oracle/_ref/launcher`` -- the reference's own timing launcher, compiled with hipcc straight
  from ``/root/reference/launcher.cpp`` (its single source file; no other reference file is
  built or copied). Built only where the reference tree is mounted; the binary travels with the
  tree so the GPU box can run the build's code object through the unmodified reference caller.
"""
from __future__ import annotations

import os
import shutil
import subprocess

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
BUILD_DIR = os.path.join(ORACLE_DIR, "_build")
REF_DIR = os.path.join(ORACLE_DIR, "_ref")
C_SO = os.path.join(BUILD_DIR, "libvark_oracle_c.so")
REF_LAUNCHER_SRC = "/root/reference/launcher.cpp"
REF_LAUNCHER = os.path.join(REF_DIR, "launcher")


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{r.stderr}")


def build_c(verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = C_SO + ".tmp"
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", os.path.join(ORACLE_DIR, "vark_oracle.c"),
          "-o", tmp, "-lm"], verbose)
    os.replace(tmp, C_SO)
    return C_SO


def build_ref_launcher(verbose: bool = False) -> str | None:
    if not os.path.exists(REF_LAUNCHER_SRC):
        return None
    os.makedirs(REF_DIR, exist_ok=True)
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    hipcc = os.path.join(rocm, "bin", "hipcc")
    hipcc = hipcc if os.path.exists(hipcc) else (shutil.which("hipcc") or "hipcc")
    tmp = REF_LAUNCHER + ".tmp"
    _run([hipcc, "-O3", "-o", tmp, REF_LAUNCHER_SRC], verbose)
    os.replace(tmp, REF_LAUNCHER)
    return REF_LAUNCHER


def build_all(verbose: bool = False):
    return build_c(verbose), build_ref_launcher(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
