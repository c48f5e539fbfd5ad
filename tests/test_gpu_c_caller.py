"""The library from a C/C++ caller (tests/c_caller/c_abi_caller.cpp, built by
tests/c_caller/build.py during the package build): headers from include/, -lggemm_vark, hipMalloc'd
buffers, the null stream -- the way the reference's launcher.cpp or a C++ framework calls it. The
program checks the ABI version, the reference-signature wgrad on the 192-row and a wide-tile
kernel, the fp32 main-grad accumulation (bit for bit C0 + result) and the persistent GEMM on
contiguous K = 2880 rows against the oracle's C restatement, and exits 0 only if every check
passes."""
import os
import subprocess

import pytest

from conftest import ROOT

EXE = os.path.join(ROOT, "tests", "c_caller", "_build", "c_abi_caller")


@pytest.mark.gpu
def test_c_caller(cuda):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is missing: run `python __graft_entry__.py build`")
    print("[gpu-case] C/C++ caller of libggemm_vark.so", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=240)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().splitlines()[-1] == "PASSED: 0 failed check(s)"
    assert r.stdout.count("\nok ") + r.stdout.startswith("ok ") == 7


def test_c_caller_links_the_in_tree_library():
    """CPU: the program resolves libggemm_vark.so to this tree's build (an $ORIGIN-relative rpath)."""
    if not os.path.exists(EXE):
        pytest.skip("c_abi_caller not built")
    out = subprocess.run(["ldd", EXE], capture_output=True, text=True, timeout=60).stdout
    line = next(l for l in out.splitlines() if "libggemm_vark.so" in l)
    assert os.path.realpath(line.split("=>")[1].split("(")[0].strip()) == \
        os.path.realpath(os.path.join(ROOT, "ggemm-asm_amd", "lib", "libggemm_vark.so"))
