"""In-tree build of the HIP artefacts for gfx950.

* ``lib/libggemm_vark.so`` -- the extern "C" launcher library: the variable-K wgrad kernels
  (tensorwise, K=32-MFMA, MXFP8; include/ggemm_vark.h), the persistent fwd/dgrad grouped GEMM
  (include/ggemm_persistent.h) and the FP8 quantization producer (include/ggemm_quant.h).
* ``lib/variable_k_wgrad.co`` -- the drop-in code object exporting only
  ``_grouped_variable_k_gemm_kernel`` with the reference kernarg layout.
* ``lib/persistent_e4m3.co`` / ``lib/persistent_e5m2.co`` -- drop-in code objects exporting only
  ``_grouped_fp8_persistent_gemm_kernel`` (e4m3 A for the forward sites, e5m2 A for dgrad).
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
PERSISTENT_CO_PATHS = {"e4m3": os.path.join(LIB_DIR, "persistent_e4m3.co"),
                       "e5m2": os.path.join(LIB_DIR, "persistent_e5m2.co")}
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


def generate_wide_asm() -> str:
    """Rewrite csrc/vark_wide_asm.inc (the wide-tile kernel's per-tile assembly) from its generator."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("gen_vark_wide", os.path.join(CSRC, "gen_vark_wide.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.main()
    return mod.OUT


def build_so(verbose: bool = False) -> str:
    generate_wide_asm()
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = SO_PATH + ".tmp"
    _run([hipcc(), *DEVICE_FLAGS, "-fPIC", "-shared", os.path.join(CSRC, "vark_capi.hip"),
          os.path.join(CSRC, "persistent_capi.hip"), os.path.join(CSRC, "quant_capi.hip"), "-o", tmp], verbose)
    os.replace(tmp, SO_PATH)
    return SO_PATH


def _build_raw_co(src: str, out: str, defines: list[str], verbose: bool) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = out + ".tmp"
    # a raw AMDGPU ELF (not a clang offload bundle), like the reference's code objects
    _run([hipcc(), *DEVICE_FLAGS, *defines, "--cuda-device-only", "--no-gpu-bundle-output",
          os.path.join(CSRC, src), "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


def build_co(verbose: bool = False) -> str:
    return _build_raw_co("vark_co.hip", CO_PATH, [], verbose)


def build_persistent_co(verbose: bool = False) -> dict:
    for fmt, path in PERSISTENT_CO_PATHS.items():
        _build_raw_co("persistent_co.hip", path, [f"-DGGEMM_A_E5M2={int(fmt == 'e5m2')}"], verbose)
    return dict(PERSISTENT_CO_PATHS)


SANITIZE_DIR = os.path.join(os.path.dirname(PKG_DIR), "_build", "sanitize")


def sanitizer_runtime() -> str:
    """clang's AddressSanitizer runtime (it carries the UBSan handlers too): preloaded into a
    process that loads a host-sanitized build."""
    llvm = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm")
    r = subprocess.run([os.path.join(llvm, "bin", "clang"), "-print-file-name=libclang_rt.asan-x86_64.so"],
                       capture_output=True, text=True)
    path = r.stdout.strip()
    if r.returncode != 0 or not os.path.isabs(path) or not os.path.exists(path):
        import glob
        hits = sorted(glob.glob(os.path.join(llvm, "lib", "clang", "*", "lib", "linux", "libclang_rt.asan-x86_64.so")))
        path = hits[-1] if hits else ""
    return path


def build_host_sanitized(verbose: bool = False) -> dict:
    """Host-side AddressSanitizer + UndefinedBehaviorSanitizer builds for the CPU tests: the
    library (its C ABI validation and launch code instrumented; device code built as usual, GPU
    sanitizers are not used) and the oracle's C restatement, both against clang's shared sanitizer
    runtime. Outputs under _build/sanitize/."""
    os.makedirs(SANITIZE_DIR, exist_ok=True)
    lib = os.path.join(SANITIZE_DIR, "libggemm_vark.so")
    host = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=undefined"]
    _run([hipcc(), *DEVICE_FLAGS, "-g", "-fPIC", "-shared", "-shared-libsan", *host,
          os.path.join(CSRC, "vark_capi.hip"), os.path.join(CSRC, "persistent_capi.hip"),
          os.path.join(CSRC, "quant_capi.hip"), "-o", lib + ".tmp"], verbose)
    os.replace(lib + ".tmp", lib)
    clang = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "clang")
    oracle_c = os.path.join(os.path.dirname(PKG_DIR), "oracle", "vark_oracle.c")
    orc = os.path.join(SANITIZE_DIR, "libvark_oracle_c.so")
    _run([clang, "-O1", "-g", "-std=c11", "-fPIC", "-shared", "-shared-libsan", "-fsanitize=address,undefined",
          "-fno-omit-frame-pointer", "-fno-sanitize-recover=undefined", oracle_c, "-o", orc + ".tmp", "-lm"], verbose)
    os.replace(orc + ".tmp", orc)
    return {"library": lib, "oracle_c": orc, "runtime": sanitizer_runtime()}


def build_all(verbose: bool = False) -> tuple[str, str]:
    so, co = build_so(verbose), build_co(verbose)
    build_persistent_co(verbose)
    return so, co


if __name__ == "__main__":
    build_all(verbose=True)
