"""Host-side AddressSanitizer / UndefinedBehaviorSanitizer run (CPU only).

The library's C ABI validation and launch code and the oracle's C restatement are rebuilt with
host ASan + UBSan (ggemm_asm_amd.build.build_host_sanitized; device code is built as usual -- GPU
sanitizers are not used), and the CPU tests that drive them -- every validation path of the three
C ABIs with unreachable device pointers, the offset checker on host arrays, the C oracle against
the numpy one -- run again in a child process against those builds with the sanitizer runtime
preloaded. Any report (heap/stack overflow, use after free, signed overflow, misaligned access,
...) aborts the child and fails this test.
"""
import os
import subprocess
import sys

import pytest

from conftest import ROOT

TESTS = ["tests/test_capi.py", "tests/test_persistent_host.py", "tests/test_quant_host.py",
         "tests/test_oracle.py::test_c_oracle_decoders_match_tables",
         "tests/test_oracle.py::test_c_oracle_agrees_with_numpy_oracle"]


def test_host_code_under_asan_ubsan(pkg):
    from ggemm_asm_amd import build
    if not os.path.exists(build.hipcc()):
        pytest.skip("hipcc not available")
    out = build.build_host_sanitized()
    if not out["runtime"]:
        pytest.skip("clang sanitizer runtime not found")
    env = dict(os.environ, GGEMM_VARK_LIBRARY=out["library"], GGEMM_ORACLE_C_LIBRARY=out["oracle_c"],
               LD_PRELOAD=out["runtime"], ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    # the child first shows that the sanitized builds are the ones mapped into it
    probe = ("import sys; sys.path[:0] = ['.', 'tests']; import ctypes;"
             "from __graft_entry__ import load_package; pkg = load_package(); pkg.load_library();"
             "from test_oracle import _c_oracle; _c_oracle();"
             "maps = open('/proc/self/maps').read();"
             f"assert {out['library']!r} in maps and {out['oracle_c']!r} in maps and 'asan' in maps, 'not loaded'")
    r = subprocess.run([sys.executable, "-c", probe], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu", *TESTS],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    log = r.stdout[-3000:] + r.stderr[-3000:]
    assert r.returncode == 0, log
    assert "AddressSanitizer" not in log and "runtime error:" not in log, log
