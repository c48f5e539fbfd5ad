"""Code-object launch harness: drives the build's `.co` files the way the reference drives its own.

Mirrors the reference's HIP module path (reference bench.py:43-143 ``load_kernel`` /
``_detect_kernel_name`` / ``unload_kernel``; bench.py:288-309,364-413 the kernelParams array
of ``prepare_variable_k_args`` / ``launch_variable_k_kernel``; bench.py:312-361
``prepare_persistent_args`` / ``launch_persistent_kernel``; launcher.cpp:16-33,123-171 the
96-byte ``KernelArgs`` record passed with HIP_LAUNCH_PARAM_BUFFER_POINTER). It exists to show
the build's code objects are drop-ins for that launch surface; the library entry points in
``vark.py`` and ``persistent.py`` are the normal way to call the kernels.
"""
from __future__ import annotations

import ctypes
import os
import struct

import torch

KERNEL_NAME = "_grouped_variable_k_gemm_kernel"
PERSISTENT_KERNEL_NAME = "_grouped_fp8_persistent_gemm_kernel"
BLOCK = 512
SHARED_MEM = 65536
KERNARG_SIZE = 96

_hip = None


def load_hip():
    global _hip
    if _hip is not None:
        return _hip
    lib = None
    for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6"):
        try:
            lib = ctypes.CDLL(name)
            break
        except OSError:
            continue
    if lib is None:
        lib = ctypes.CDLL(os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib", "libamdhip64.so"))
    vp = ctypes.c_void_p
    lib.hipModuleLoadData.argtypes = [ctypes.POINTER(vp), vp]
    lib.hipModuleLoadData.restype = ctypes.c_int
    lib.hipModuleGetFunction.argtypes = [ctypes.POINTER(vp), vp, ctypes.c_char_p]
    lib.hipModuleGetFunction.restype = ctypes.c_int
    lib.hipModuleLaunchKernel.argtypes = [vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                          ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, vp,
                                          ctypes.POINTER(vp), ctypes.POINTER(vp)]
    lib.hipModuleLaunchKernel.restype = ctypes.c_int
    lib.hipModuleUnload.argtypes = [vp]
    lib.hipModuleUnload.restype = ctypes.c_int
    lib.hipGetErrorString.argtypes = [ctypes.c_int]
    lib.hipGetErrorString.restype = ctypes.c_char_p
    lib.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
    lib.hipEventCreate.restype = ctypes.c_int
    lib.hipEventRecord.argtypes = [vp, vp]
    lib.hipEventRecord.restype = ctypes.c_int
    lib.hipEventSynchronize.argtypes = [vp]
    lib.hipEventSynchronize.restype = ctypes.c_int
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
    lib.hipEventElapsedTime.restype = ctypes.c_int
    lib.hipEventDestroy.argtypes = [vp]
    lib.hipEventDestroy.restype = ctypes.c_int
    lib.hipDeviceSynchronize.argtypes = []
    lib.hipDeviceSynchronize.restype = ctypes.c_int
    _hip = lib
    return lib


def time_null_stream(launch, iters: int, warmup: int) -> float:
    """Average ms per launch of ``launch`` (which enqueues on the null stream, as the reference's
    launches do) from two HIP events recorded on the null stream around ``iters`` back-to-back
    launches after ``warmup`` untimed ones (reference bench.py:768-801, launcher.cpp:149-176)."""
    hip = load_hip()
    for _ in range(warmup):
        launch()
    check_hip(hip.hipDeviceSynchronize(), "synchronizing before timing")
    ev = [ctypes.c_void_p(), ctypes.c_void_p()]
    for e in ev:
        check_hip(hip.hipEventCreate(ctypes.byref(e)), "creating a timing event")
    try:
        check_hip(hip.hipEventRecord(ev[0], None), "recording the start event")
        for _ in range(iters):
            launch()
        check_hip(hip.hipEventRecord(ev[1], None), "recording the stop event")
        check_hip(hip.hipEventSynchronize(ev[1]), "waiting for the stop event")
        ms = ctypes.c_float()
        check_hip(hip.hipEventElapsedTime(ctypes.byref(ms), ev[0], ev[1]), "reading the elapsed time")
    finally:
        for e in ev:
            hip.hipEventDestroy(e)
    return ms.value / max(iters, 1)


def check_hip(err: int, msg: str = "") -> None:
    if err != 0:
        raise RuntimeError(f"HIP error {err} ({load_hip().hipGetErrorString(err)}): {msg}")


# ----------------------------------------------------------------------------- ELF symbols

def elf_global_functions(data: bytes) -> list[str]:
    """Names of FUNC GLOBAL symbols of an ELF64 little-endian object (what the reference reads
    with ``llvm-readelf -s``, bench.py:118-131), parsed directly from the section headers."""
    if data[:4] != b"\x7fELF" or data[4] != 2 or data[5] != 1:
        raise ValueError("not an ELF64 little-endian object")
    e_shoff = struct.unpack_from("<Q", data, 0x28)[0]
    e_shentsize, e_shnum = struct.unpack_from("<HH", data, 0x3A)
    names = []
    for i in range(e_shnum):
        sh = e_shoff + i * e_shentsize
        sh_type = struct.unpack_from("<I", data, sh + 4)[0]
        if sh_type not in (2, 11):  # SHT_SYMTAB, SHT_DYNSYM
            continue
        sh_offset, sh_size = struct.unpack_from("<QQ", data, sh + 0x18)
        sh_link = struct.unpack_from("<I", data, sh + 0x28)[0]
        sh_entsize = struct.unpack_from("<Q", data, sh + 0x38)[0] or 24
        strtab = e_shoff + sh_link * e_shentsize
        str_off = struct.unpack_from("<Q", data, strtab + 0x18)[0]
        for j in range(sh_size // sh_entsize):
            st = sh_offset + j * sh_entsize
            st_name, st_info = struct.unpack_from("<IB", data, st)
            if (st_info & 0xF) == 2 and (st_info >> 4) == 1:  # STT_FUNC, STB_GLOBAL
                end = data.index(b"\0", str_off + st_name)
                names.append(data[str_off + st_name:end].decode())
    return names


def detect_kernel_name(data: bytes) -> str:
    for name in elf_global_functions(data):
        if name.startswith("_grouped"):
            return name
    raise RuntimeError("no FUNC GLOBAL symbol starting with _grouped in the code object")


# ----------------------------------------------------------------------------- module API

def load_kernel(co_path: str, kernel_name: str | None = None):
    """Load a code object; returns (module, function, kernel_name)."""
    hip = load_hip()
    with open(co_path, "rb") as f:
        data = f.read()
    module = ctypes.c_void_p()
    check_hip(hip.hipModuleLoadData(ctypes.byref(module), data), f"loading {co_path}")
    name = kernel_name or detect_kernel_name(data)
    func = ctypes.c_void_p()
    check_hip(hip.hipModuleGetFunction(ctypes.byref(func), module, name.encode()), f"getting {name}")
    return module, func, name


def unload_kernel(module) -> None:
    load_hip().hipModuleUnload(module)


def _llvm_tool(name: str) -> str:
    cand = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", name)
    return cand if os.path.exists(cand) else name


_INFO_KEYS = ("vgpr_count", "agpr_count", "sgpr_count", "vgpr_spill_count", "sgpr_spill_count",
              "group_segment_fixed_size", "private_segment_fixed_size", "kernarg_segment_size",
              "max_flat_workgroup_size", "wavefront_size")


def kernel_info(co_path: str) -> dict:
    """Resource usage of a code object built here, per kernel, the counterpart of the reference's
    ``print_kernel_info`` (bench.py:544-589): registers, spills, LDS, scratch and kernarg bytes from
    the AMDGPU metadata note (llvm-readelf --notes), plus instruction and MFMA counts from the
    disassembly (llvm-objdump). Only for this build's own code objects."""
    import re
    import subprocess
    notes = subprocess.run([_llvm_tool("llvm-readelf"), "--notes", co_path], capture_output=True, text=True,
                           timeout=60).stdout
    kernels = {}
    for chunk in re.split(r"\n\s*- \.agpr_count:", notes)[1:]:
        chunk = ".agpr_count:" + chunk
        name = re.search(r"\.name:\s+(\S+)", chunk).group(1)
        info = {k: int(m.group(1)) for k in _INFO_KEYS
                if (m := re.search(rf"\.{k}:\s+(\d+)", chunk))}
        kernels[name] = info
    dis = subprocess.run([_llvm_tool("llvm-objdump"), "-d", "--mcpu=gfx950", co_path], capture_output=True, text=True,
                         timeout=120).stdout
    current = None
    for line in dis.splitlines():
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            current = kernels.setdefault(m.group(1), {})
            current.update(instructions=0, mfma=0, s_nop=0, lds_dma=0)
            continue
        ins = line.split("//")[0].strip()
        if current is None or not ins or not line[:1].isspace():
            continue
        current["instructions"] += 1
        current["mfma"] += ins.startswith("v_mfma")
        current["s_nop"] += ins.startswith("s_nop")
        current["lds_dma"] += ins.startswith("buffer_load") and ins.endswith(" lds")
    return {"file": co_path, "bytes": os.path.getsize(co_path), "kernels": kernels}


def get_num_cus(device: int = 0) -> int:
    return torch.cuda.get_device_properties(device).multi_processor_count


# Byte offsets of the 16 kernarg fields (six pointers, eight int32, two scratch pointers; reference
# launcher.cpp:16-33): hipModuleLaunchKernel's kernelParams entry i points at field i.
_FIELD_OFFSETS = tuple(range(0, 48, 8)) + tuple(range(48, 80, 4)) + (80, 88)


def _kernel_params(record: bytes):
    """kernelParams array over one 96-byte kernarg record; the buffer must outlive the launch."""
    buf = ctypes.create_string_buffer(record, KERNARG_SIZE)
    base = ctypes.addressof(buf)
    return (ctypes.c_void_p * len(_FIELD_OFFSETS))(*(base + o for o in _FIELD_OFFSETS)), buf


def prepare_variable_k_args(func, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N,
                            num_sms, shared_mem=SHARED_MEM):
    """Closure launching with a kernelParams array on the null stream (bench.py:364-402)."""
    hip = load_hip()
    params, storage = _kernel_params(kernarg_buffer(lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N))

    def launch():
        check_hip(hip.hipModuleLaunchKernel(func, num_sms, 1, 1, BLOCK, 1, 1, shared_mem, None, params, None),
                  "launching variable-K kernel")

    return launch, storage


def launch_variable_k_kernel(func, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, num_sms,
                             shared_mem=SHARED_MEM):
    launch, _keep = prepare_variable_k_args(func, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M,
                                            OUT_N, num_sms, shared_mem)
    launch()


def persistent_kernarg_buffer(a, b, out, a_scale, b_scale, group_offs, G, N, K) -> bytes:
    """The persistent kernel's 96-byte record (reference bench.py:317-336): strides from the
    tensors, b as [G, N, K], out as [M, N]."""
    return struct.pack("<6Q8i2Q", a.data_ptr(), b.data_ptr(), out.data_ptr(), a_scale.data_ptr(),
                       b_scale.data_ptr(), group_offs.data_ptr(), G, N, K, a.stride(0), b.stride(0),
                       b.stride(1), out.stride(0), out.stride(1), 0, 0)


def prepare_persistent_args(func, a, b, out, a_scale, b_scale, group_offs, G, N, K, num_sms,
                            shared_mem=SHARED_MEM):
    """Closure launching the persistent fwd/dgrad kernel on the null stream (bench.py:312-351)."""
    hip = load_hip()
    params, storage = _kernel_params(persistent_kernarg_buffer(a, b, out, a_scale, b_scale, group_offs, G, N, K))

    def launch():
        check_hip(hip.hipModuleLaunchKernel(func, num_sms, 1, 1, BLOCK, 1, 1, shared_mem, None, params, None),
                  "launching persistent kernel")

    return launch, storage


def launch_persistent_kernel(func, a, b, out, a_scale, b_scale, group_offs, G, N, K, num_sms,
                             shared_mem=SHARED_MEM):
    launch, _keep = prepare_persistent_args(func, a, b, out, a_scale, b_scale, group_offs, G, N, K, num_sms,
                                            shared_mem)
    launch()


def kernarg_buffer(lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N) -> bytes:
    """The 96-byte KernelArgs record of launcher.cpp:16-33: six pointers, eight int32, two null
    scratch pointers."""
    return struct.pack("<6Q8i2Q", lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), lhs_scale.data_ptr(),
                       rhs_scale.data_ptr(), group_offs.data_ptr(), G, OUT_M, OUT_N, lhs.stride(0),
                       rhs.stride(0), out.stride(0), out.stride(1), out.stride(2), 0, 0)


def launch_with_kernarg_buffer(func, kernarg: bytes, num_sms, shared_mem=SHARED_MEM) -> None:
    """Launch with HIP_LAUNCH_PARAM_BUFFER_POINTER (launcher.cpp:142-147)."""
    if len(kernarg) != KERNARG_SIZE:
        raise ValueError("kernarg record must be 96 bytes")
    hip = load_hip()
    buf = ctypes.create_string_buffer(kernarg, KERNARG_SIZE)
    size = ctypes.c_size_t(KERNARG_SIZE)
    extra = (ctypes.c_void_p * 5)(ctypes.c_void_p(1), ctypes.cast(buf, ctypes.c_void_p), ctypes.c_void_p(2),
                                  ctypes.cast(ctypes.pointer(size), ctypes.c_void_p), ctypes.c_void_p(3))
    check_hip(hip.hipModuleLaunchKernel(func, num_sms, 1, 1, BLOCK, 1, 1, shared_mem, None, None, extra),
              "launching with kernarg buffer")
