"""CPU checks of the C-ABI library and the drop-in code object (no kernel launches).

Argument validation runs before any HIP call, so invalid-argument paths are exercised here with
fake (never dereferenced) pointers.
"""
import ctypes
import os
import re
import shutil
import subprocess

import pytest
import torch

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ggemm_vark.h")


def _header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\s*\*?\s*(ggemm_vark_\w+)\s*\(", text, re.M)))


def test_bf16_kernel_selection(pkg):
    """The bf16 entry points take a wide-tile kernel for large OUT_M: 320 x 320 where both output
    dims are multiples of 320, else 256 x 384 with OUT_N a multiple of 384, with a 16-byte aligned
    C; every other shape keeps the 192-row-tile kernel."""
    lib = pkg.load_library()
    assert lib.ggemm_vark_bf16_kernel(2880, 5760, 5760, 4096) == 320
    assert lib.ggemm_vark_bf16_kernel(2880, 2880, 2880, 4096) == 320
    assert lib.ggemm_vark_bf16_kernel(1024, 384, 384, 4096) == 256
    assert lib.ggemm_vark_bf16_kernel(3072, 5376, 5376, 4096) == 256
    assert lib.ggemm_vark_bf16_kernel(2048, 2000, 2000, 4096) == 0      # neither tile divides OUT_N
    assert lib.ggemm_vark_bf16_kernel(1008, 5760, 5760, 4096) == 0      # small OUT_M
    assert lib.ggemm_vark_bf16_kernel(2880, 5760, 5760, 4104) == 0      # C only 8-byte aligned
    assert lib.ggemm_vark_bf16_kernel(2880, 5760, 5768, 4096) == 320    # padded rows on 16 bytes
    assert lib.ggemm_vark_bf16_kernel(2880, 5760, 5764, 4096) == 0      # rows on 8 bytes: 192-row kernel
    assert lib.ggemm_vark_bf16_kernel(65536, 384, 65536, 4096) == 0     # group past 32-bit offsets
    assert pkg.bf16_kernel(2880, 5760) == "wide320" and pkg.bf16_kernel(1024, 768) == "wide256"
    assert pkg.bf16_kernel(1000, 2880) == "192-row"


def test_library_exports_every_header_symbol(pkg):
    lib = pkg.load_library()
    names = _header_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    from ggemm_asm_amd import _lib
    assert set(names) == set(_lib.EXPORTS)


def test_abi_version_and_geometry(pkg):
    lib = pkg.load_library()
    ver = int(re.search(r"#define GGEMM_VARK_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.ggemm_vark_abi_version() == ver
    assert pkg.launch_geometry(5760) == {"block_threads": 512, "dynamic_lds": 65536, "tile_m": 192,
                                         "tile_n": 384, "k_step": 128}
    # 384-wide tiles also when at least four fit and the last is at least half full
    assert pkg.launch_geometry(2880)["tile_n"] == 384
    assert [pkg.launch_geometry(n)["tile_n"] for n in (640, 1344, 1536 + 191, 1536 + 192, 320)] == [320, 320, 320, 384, 320]


def _offs(vals):
    a = (ctypes.c_int64 * len(vals))(*vals)
    return a


@pytest.mark.parametrize("vals,M,mx,rc", [
    ([0, 96, 256, 256, 512], 512, 0, 0),
    ([0, 96, 256, 256, 512], 511, 0, -5),     # past M_total
    ([1, 96, 256], 512, 0, -5),               # not 0-based
    ([0, 96, 90, 512], 512, 0, -5),           # decreasing
    ([0, 64, 64, 160, 205], 205, 1, 0),       # MX: starts aligned, ragged last group allowed
    ([0, 96, 100, 512], 512, 1, -7),          # MX: group 2 starts at 100
])
def test_check_offsets(pkg, vals, M, mx, rc):
    lib = pkg.load_library()
    assert lib.ggemm_vark_check_offsets(_offs(vals), len(vals) - 1, M, mx) == rc


def test_strerror(pkg):
    lib = pkg.load_library()
    for code in range(-7, 1):
        s = lib.ggemm_vark_strerror(code).decode()
        assert s and s != "unknown error"


FAKE = 0x100000  # 16-byte aligned, never dereferenced: validation fails before any HIP call


def _call(lib, **kw):
    a = dict(lhs=FAKE, rhs=FAKE, out=FAKE, ls=FAKE, rs=FAKE, offs=FAKE, G=32, OUT_M=2880, OUT_N=5760,
             slm=2880, srm=5760, scg=2880 * 5760, scm=5760, scn=1)
    a.update(kw)
    return lib.ggemm_vark_wgrad_fp8(a["lhs"], a["rhs"], a["out"], a["ls"], a["rs"], a["offs"], a["G"], a["OUT_M"],
                                    a["OUT_N"], a["slm"], a["srm"], a["scg"], a["scm"], a["scn"], None)


@pytest.mark.parametrize("kw,rc", [
    (dict(lhs=0), -1), (dict(offs=0), -1), (dict(G=0), -2), (dict(OUT_M=100, slm=100), -2),
    (dict(OUT_N=-16), -2), (dict(scn=2), -3), (dict(slm=2800), -3), (dict(srm=5768), -3),
    (dict(scm=5762), -3), (dict(scg=100), -3), (dict(lhs=FAKE + 8), -4), (dict(out=FAKE + 2), -4),
    # more than 2^30 tiles of at most 192 x 320: 32-bit tile indices would overflow
    (dict(G=(1 << 30) // 270 + 1), -2),
])
def test_validation_rejects(pkg, kw, rc):
    assert _call(pkg.load_library(), **kw) == rc


@pytest.mark.parametrize("mode,kw,rc", [
    (3, {}, -8), (-1, {}, -8), (1, dict(out=FAKE + 8), -4), (2, dict(out=FAKE + 8), -4), (1, dict(scn=2), -3),
    (2, dict(scm=5762), -3), (1, dict(lhs=0), -1),
    # a negative token count, in every output mode
    (0, dict(M=-1), -2), (1, dict(M=-1), -2), (2, dict(M=-5), -2),
])
def test_fp32_out_validation_rejects(pkg, mode, kw, rc):
    lib = pkg.load_library()
    a = dict(lhs=FAKE, rhs=FAKE, out=FAKE, ls=FAKE, rs=FAKE, offs=FAKE, G=32, OUT_M=2880, OUT_N=5760,
             slm=2880, srm=5760, scg=2880 * 5760, scm=5760, scn=1, M=131072)
    a.update(kw)
    assert lib.ggemm_vark_wgrad_fp8_out(a["lhs"], a["rhs"], a["out"], a["ls"], a["rs"], a["offs"], a["G"], a["OUT_M"],
                                        a["OUT_N"], a["slm"], a["srm"], a["scg"], a["scm"], a["scn"], mode, a["M"],
                                        None) == rc


def test_mx_validation_rejects(pkg):
    lib = pkg.load_library()
    args = [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 128, 64, 128, 64 * 128, 128, 1]
    assert lib.ggemm_vark_wgrad_mxfp8(*args, 60, 128, 512, None) == -3      # scale stride < OUT_M
    assert lib.ggemm_vark_wgrad_mxfp8(*args[:3], FAKE + 4, *args[4:], 64, 128, 512, None) == -4
    assert lib.ggemm_vark_wgrad_mxfp8(*args, 64, 128, -1, None) == -2       # negative token count


def test_integer_arguments_out_of_range_raise(pkg):
    """A size or stride beyond a parameter's width raises in the binding. Plain ctypes integer
    types keep the low bits: N = 2**32 + 320 would reach the library as N = 320 (the wide kernel's
    shape), and a row stride of 2**32 + 5762 as 5762."""
    import numpy as np

    lib = pkg.load_library()
    assert lib.ggemm_persistent_selected_kernel(320, 2880, 2880, 2880, 320) == 2
    with pytest.raises(ctypes.ArgumentError, match="does not fit"):
        lib.ggemm_persistent_selected_kernel((1 << 32) + 320, 2880, 2880, 2880, 320)
    with pytest.raises(ctypes.ArgumentError, match="does not fit"):
        _call(lib, scm=(1 << 32) + 5762)
    with pytest.raises(ctypes.ArgumentError, match="does not fit"):
        lib.ggemm_vark_check_offsets(None, 1, 1 << 63, 0)
    with pytest.raises(ctypes.ArgumentError):   # a float is not a size
        _call(lib, G=32.0)
    assert _call(lib, scm=np.int64(5762), G=np.int32(32)) == -3   # numpy integers pass as ints


def test_python_op_refuses_rows_short_of_their_stride(pkg):
    """An operand whose last row ends before its row stride (an as_strided view over a buffer one
    padding short) is refused: the kernels may read a row's padding. A view into a tensor of full
    rows passes that check (and, on the CPU, stops at the device check)."""
    buf = torch.zeros(63 * 96 + 64, dtype=torch.uint8)
    short = torch.as_strided(buf, (64, 64), (96, 1))
    full = torch.zeros(64, 96, dtype=torch.uint8)[:, :64]
    rhs = torch.zeros(64, 128, dtype=torch.uint8)
    s = torch.tensor(1.0)
    offs = torch.tensor([0, 64], dtype=torch.int64)
    with pytest.raises(ValueError, match="row stride"):
        pkg.grouped_gemm_fp8_tensorwise_variable_k(short, rhs, s, s, offs)
    with pytest.raises(ValueError, match="row stride"):
        pkg.grouped_gemm_fp8_tensorwise_variable_k(rhs, short, s, s, offs)
    with pytest.raises(ValueError, match="gfx950 GPU only"):
        pkg.grouped_gemm_fp8_tensorwise_variable_k(full, rhs, s, s, offs)


def test_python_op_refuses_cpu_tensors(pkg):
    lhs = torch.zeros(64, 64, dtype=torch.uint8)
    rhs = torch.zeros(64, 128, dtype=torch.uint8)
    s = torch.tensor(1.0)
    offs = torch.tensor([0, 64], dtype=torch.int64)
    with pytest.raises(ValueError, match="gfx950 GPU only"):
        pkg.grouped_gemm_fp8_tensorwise_variable_k(lhs, rhs, s, s, offs)


def test_torch_op_meta_shape(pkg):
    lhs = torch.empty(512, 64, dtype=torch.uint8, device="meta")
    rhs = torch.empty(512, 128, dtype=torch.uint8, device="meta")
    s = torch.empty((), dtype=torch.float32, device="meta")
    offs = torch.empty(5, dtype=torch.int64, device="meta")
    out = torch.ops.ggemm.variable_k_wgrad_fp8(lhs, rhs, s, s, offs)
    assert out.shape == (4, 64, 128) and out.dtype == torch.bfloat16


# ----------------------------------------------------------------------------- code object

def _readelf():
    for c in ("/opt/rocm/llvm/bin/llvm-readelf", shutil.which("llvm-readelf")):
        if c and os.path.exists(c):
            return c
    pytest.skip("llvm-readelf not available")


def test_code_object_symbol_and_kernarg_layout(pkg):
    from ggemm_asm_amd import harness
    data = open(pkg.CODE_OBJECT_PATH, "rb").read()
    assert data[:4] == b"\x7fELF"
    assert set(harness.elf_global_functions(data)) == {"_grouped_variable_k_gemm_kernel"}
    assert harness.detect_kernel_name(data) == "_grouped_variable_k_gemm_kernel"
    notes = subprocess.run([_readelf(), "--notes", pkg.CODE_OBJECT_PATH], capture_output=True, text=True,
                           timeout=30).stdout
    assert re.search(r"\.kernarg_segment_size:\s+96\b", notes)
    assert re.search(r"\.max_flat_workgroup_size:\s+512\b", notes)
    offs = [int(x) for x in re.findall(r"\.offset:\s+(\d+)", notes)]
    sizes = [int(x) for x in re.findall(r"\.size:\s+(\d+)", notes)]
    kinds = re.findall(r"\.value_kind:\s+(\w+)", notes)
    # reference launcher.cpp:16-33: 6 pointers, 8 int32 at 48..76, 2 pointers at 80/88
    assert offs == [0, 8, 16, 24, 32, 40, 48, 52, 56, 60, 64, 68, 72, 76, 80, 88]
    assert sizes == [8] * 6 + [4] * 8 + [8, 8]
    assert kinds == ["global_buffer"] * 6 + ["by_value"] * 8 + ["global_buffer"] * 2
    lds = int(re.search(r"\.group_segment_fixed_size:\s+(\d+)", notes).group(1))
    assert lds + 65536 <= 160 * 1024   # static LDS + the launch's 64 KiB dynamic fit gfx950's 160 KiB


def _vgpr_set(op):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", op) or re.fullmatch(r"v(\d+)", op)
    if not m:
        return set()
    lo = int(m.group(1))
    hi = int(m.group(2)) if m.lastindex == 2 else lo
    return set(range(lo, hi + 1))


def test_wide_store_data_hazard(pkg):
    """gfx950: a VALU may not write the data VGPRs of a preceding VMEM store wider than 8 bytes
    within two wait states. The compiler pads the stores it emits; this guards against a wide
    store slipping in from inline asm (it corrupted the first dword of stored chunks)."""
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not available")
    txt = subprocess.run([objdump, "-d", "--mcpu=gfx950", pkg.CODE_OBJECT_PATH], capture_output=True,
                         text=True, timeout=60).stdout
    ins = [l.split("//")[0].strip() for l in txt.splitlines() if l.startswith("\t") or l.startswith("  ")]
    ins = [i for i in ins if i]
    n_wide = 0
    for k, i in enumerate(ins):
        m = re.match(r"(global|buffer|flat)_store_dword(x3|x4)\s+(\S+),\s*(\S+)", i)
        if not m:
            continue
        n_wide += 1
        data = _vgpr_set(m.group(4).rstrip(",") if m.group(1) == "global" else m.group(3).rstrip(","))
        states = 0
        for nxt in ins[k + 1:k + 4]:
            if states >= 2:
                break
            nop = re.match(r"s_nop\s+(\d+)", nxt)
            if nop:
                states += int(nop.group(1)) + 1
                continue
            if nxt.startswith("v_"):
                dst = nxt.split()[1].rstrip(",") if len(nxt.split()) > 1 else ""
                assert not (_vgpr_set(dst) & data), f"store-data hazard: {i!r} then {nxt!r}"
            states += 1
    assert n_wide >= 1


def test_tensorwise_code_object_uses_unscaled_mfma(pkg):
    """The per-tensor kernels pass constant zero scale operands so the compiler emits the unscaled
    v_mfma_f32_16x16x128_f8f6f4 (equal to scale 2^0, measured bit-identical on the GPU). A
    compiler that emitted the scaled form for them would multiply C by 2^-254: catch it here."""
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not available")
    txt = subprocess.run([objdump, "-d", "--mcpu=gfx950", pkg.CODE_OBJECT_PATH], capture_output=True,
                         text=True, timeout=60).stdout
    assert re.search(r"\bv_mfma_f32_16x16x128_f8f6f4\b", txt)
    assert "v_mfma_scale" not in txt


def test_m0_only_feeds_lds_dma(pkg):
    """The LDS-DMA loads set m0 from inline asm; nothing else in the kernels may use m0."""
    objdump = "/opt/rocm/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not available")
    txt = subprocess.run([objdump, "-d", "--mcpu=gfx950", pkg.CODE_OBJECT_PATH], capture_output=True,
                         text=True, timeout=60).stdout
    ins = [l.split("//")[0].strip() for l in txt.splitlines() if l.startswith("\t") or l.startswith("  ")]
    ins = [i for i in ins if i]
    n_dma = 0
    for k, i in enumerate(ins):
        if re.search(r"\bm0\b", i):
            assert i.startswith("s_mov_b32 m0,"), i
            assert ins[k + 1].startswith("buffer_load_dwordx4") and ins[k + 1].rstrip().endswith("lds"), ins[k + 1]
            n_dma += 1
    assert n_dma >= 8


def test_code_object_resources(pkg):
    """The drop-in wgrad code object keeps its registers: no VGPR spills and no scratch (a spill
    would put scratch traffic in the stage loop), at most 256 VGPRs (two 64-lane waves per SIMD,
    the 512-thread launch contract), the 96 KiB static LDS, the 96-byte kernarg; and it is built on
    the MFMA and LDS-DMA instructions it is designed around."""
    from ggemm_asm_amd import harness
    info = harness.kernel_info(pkg.CODE_OBJECT_PATH)["kernels"]["_grouped_variable_k_gemm_kernel"]
    assert info["vgpr_spill_count"] == 0 and info["private_segment_fixed_size"] == 0, info
    assert info["vgpr_count"] + info["agpr_count"] <= 256, info
    assert info["group_segment_fixed_size"] == 98304 and info["kernarg_segment_size"] == 96, info
    assert info["max_flat_workgroup_size"] == 512 and info["wavefront_size"] == 64, info
    assert info["mfma"] >= 36 and info["lds_dma"] >= 9, info


@pytest.mark.parametrize("mode,scm,scg,rc", [
    (0, 5764, 2880 * 5764, -4), (0, 5768, 2880 * 5768 + 4, -4), (1, 5762, 2880 * 5762, -3),
    (2, 5766, 2880 * 5766, -3),
])
def test_wide_entry_requires_16_byte_rows(pkg, mode, scm, scg, rc):
    """The forced wide-tile entry refuses C rows or groups that do not start on 16 bytes (its
    epilogue stores 16-byte row chunks): bf16 strides must be multiples of 8 elements, fp32 of 4.
    Only rejected calls here: nothing is launched."""
    lib = pkg.load_library()
    assert lib.ggemm_vark_wgrad_fp8_wide(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 32, 2880, 5760, 2880, 5760, scg, scm, 1,
                                         131072, 320, mode, None) == rc
    if mode == 0:   # the MX kernel on request applies the same rule
        assert lib.ggemm_vark_wgrad_mxfp8_tile(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 32, 2880, 5760, 2880, 5760, scg,
                                               scm, 1, 2880, 5760, 131072, 320, None) == rc
