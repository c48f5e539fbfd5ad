"""Build recipe of the C/C++ caller test program (TEST INFRASTRUCTURE ONLY).

``tests/c_caller/_build/c_abi_caller``: ``c_abi_caller.cpp`` (host C++, no device code: g++ with the
HIP runtime headers) linked against the product library ``ggemm-asm_amd/lib/libggemm_vark.so`` (found
through an $ORIGIN-relative rpath, so the tree can move) and the oracle's C restatement
``oracle/vark_oracle.c`` (the checker). Run after the library is built; ``tests/test_gpu_c_caller.py``
runs the program on the GPU.
"""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
BUILD_DIR = os.path.join(HERE, "_build")
EXE = os.path.join(BUILD_DIR, "c_abi_caller")


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"c_abi_caller build failed: {' '.join(cmd)}\n{r.stderr}")


def build(verbose: bool = False) -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    os.makedirs(BUILD_DIR, exist_ok=True)
    obj = os.path.join(BUILD_DIR, "vark_oracle.o")
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-c", os.path.join(ROOT, "oracle", "vark_oracle.c"), "-o", obj], verbose)
    tmp = EXE + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include",
          os.path.join(HERE, "c_abi_caller.cpp"), obj,
          "-L", os.path.join(ROOT, "ggemm-asm_amd", "lib"), "-lggemm_vark", f"-L{rocm}/lib", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN/../../../ggemm-asm_amd/lib", f"-Wl,-rpath,{rocm}/lib", "-lm", "-o", tmp], verbose)
    os.replace(tmp, EXE)
    return EXE


if __name__ == "__main__":
    build(verbose=True)
