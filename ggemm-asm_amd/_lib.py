"""ctypes binding of libggemm_vark.so (declarations in include/ggemm_vark.h,
include/ggemm_persistent.h and include/ggemm_quant.h)."""
from __future__ import annotations

import ctypes
import operator
import os

from . import build as _build

_lib = None


class _CheckedInt:
    """Argument type of an integer parameter: ctypes' own ``c_int32`` / ``c_int64`` keep only the
    low bits of a Python int that does not fit (2**32 + 5 arrives as 5), which would hand the
    library's validation -- and the kernel -- a different size or stride from the tensor's. This
    one raises OverflowError instead, and TypeError for a non-integer (a float)."""
    bits = 32
    ctype = ctypes.c_int32

    @classmethod
    def from_param(cls, v):
        v = operator.index(v)
        if not -(1 << (cls.bits - 1)) <= v < (1 << (cls.bits - 1)):
            raise OverflowError(f"{v} does not fit the library's {cls.bits}-bit integer parameter")
        return cls.ctype(v)


class _I32(_CheckedInt):
    pass


class _I64(_CheckedInt):
    bits = 64
    ctype = ctypes.c_int64


EXPORTS = (
    "ggemm_vark_wgrad_fp8",
    "ggemm_vark_wgrad_fp8_k32",
    "ggemm_vark_wgrad_fp8_out",
    "ggemm_vark_wgrad_fp8_wide",
    "ggemm_vark_wgrad_mxfp8",
    "ggemm_vark_wgrad_mxfp8_tile",
    "ggemm_vark_check_offsets",
    "ggemm_vark_num_cus",
    "ggemm_vark_strerror",
    "ggemm_vark_abi_version",
    "ggemm_vark_bf16_kernel",
    "ggemm_vark_launch_geometry",
)

PERSISTENT_EXPORTS = (
    "ggemm_persistent_fp8",
    "ggemm_persistent_fp8_kernel",
    "ggemm_persistent_selected_kernel",
    "ggemm_persistent_clear_tail",
    "ggemm_persistent_transpose_u8",
)

QUANT_EXPORTS = (
    "ggemm_quant_amax",
    "ggemm_quant_fp8_tensorwise",
    "ggemm_quant_fp8_tensorwise_delayed",
    "ggemm_quant_fp8_tensorwise_delayed_dev",
    "ggemm_quant_fp8_tensorwise_transpose",
    "ggemm_quant_fp8_tensorwise_transpose_delayed",
    "ggemm_quant_fp8_tensorwise_transpose_delayed_dev",
    "ggemm_quant_mxfp8_grouped",
)

# GGEMM_VARK_ABI_VERSION of include/ggemm_vark.h that these bindings are written for. Some exports
# changed signature between versions (ggemm_vark_wgrad_fp8_out and ggemm_vark_wgrad_mxfp8 took
# M_total from version 3 on), so a library of another version is refused at load.
ABI_VERSION = 9

ERRORS = {
    0: "GGEMM_OK", -1: "GGEMM_E_NULL", -2: "GGEMM_E_SHAPE", -3: "GGEMM_E_STRIDE",
    -4: "GGEMM_E_ALIGN", -5: "GGEMM_E_OFFSETS", -6: "GGEMM_E_DEVICE", -7: "GGEMM_E_MX_ALIGN",
    -8: "GGEMM_E_FORMAT",
}


class GGemmError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what} failed with {ERRORS.get(code, 'hipError')} ({code}): {strerror(code)}")


def library_path() -> str:
    """The in-tree library, or the one GGEMM_VARK_LIBRARY names (a variant build of the same
    sources, e.g. the host-sanitizer build the CPU tests run the C ABI's validation under)."""
    return os.environ.get("GGEMM_VARK_LIBRARY") or _build.SO_PATH


def load():
    """Load the in-tree library; raise if it has not been built (there is no fallback path)."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run `python __graft_entry__.py build` first "
                           "(this package has no CPU or Python fallback for the kernel)")
    lib = ctypes.CDLL(path)
    lib.ggemm_vark_abi_version.argtypes = []
    lib.ggemm_vark_abi_version.restype = ctypes.c_int32
    if lib.ggemm_vark_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {lib.ggemm_vark_abi_version()}, these bindings need "
                           f"{ABI_VERSION}: rebuild with `python __graft_entry__.py build`")
    vp, i32, i64, i64p = ctypes.c_void_p, _I32, _I64, ctypes.POINTER(ctypes.c_int64)
    tw = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp]
    for name in ("ggemm_vark_wgrad_fp8", "ggemm_vark_wgrad_fp8_k32"):
        f = getattr(lib, name)
        f.argtypes = tw
        f.restype = ctypes.c_int
    lib.ggemm_vark_wgrad_fp8_out.argtypes = tw[:-1] + [i32, i64, vp]
    lib.ggemm_vark_wgrad_fp8_out.restype = ctypes.c_int
    lib.ggemm_vark_wgrad_fp8_wide.argtypes = tw[:-1] + [i64, i32, i32, vp]
    lib.ggemm_vark_wgrad_fp8_wide.restype = ctypes.c_int
    lib.ggemm_vark_wgrad_mxfp8.argtypes = [vp, vp, vp, vp, vp, vp] + [i32] * 10 + [i64, vp]
    lib.ggemm_vark_wgrad_mxfp8.restype = ctypes.c_int
    lib.ggemm_vark_wgrad_mxfp8_tile.argtypes = [vp, vp, vp, vp, vp, vp] + [i32] * 10 + [i64, i32, vp]
    lib.ggemm_vark_wgrad_mxfp8_tile.restype = ctypes.c_int
    lib.ggemm_vark_check_offsets.argtypes = [i64p, i32, i64, i32]
    lib.ggemm_vark_check_offsets.restype = ctypes.c_int
    lib.ggemm_vark_num_cus.argtypes = [i32, ctypes.POINTER(ctypes.c_int32)]
    lib.ggemm_vark_num_cus.restype = ctypes.c_int
    lib.ggemm_vark_strerror.argtypes = [i32]
    lib.ggemm_vark_strerror.restype = ctypes.c_char_p
    lib.ggemm_vark_abi_version.argtypes = []
    lib.ggemm_vark_abi_version.restype = ctypes.c_int32
    lib.ggemm_vark_bf16_kernel.argtypes = [i32, i32, i32, vp]
    lib.ggemm_vark_bf16_kernel.restype = ctypes.c_int32
    lib.ggemm_vark_launch_geometry.argtypes = [i32] + [ctypes.POINTER(ctypes.c_int32)] * 5
    lib.ggemm_vark_launch_geometry.restype = None
    lib.ggemm_persistent_fp8.argtypes = [vp, vp, vp, vp, vp, vp] + [i32] * 9 + [i64, vp]
    lib.ggemm_persistent_fp8.restype = ctypes.c_int
    lib.ggemm_persistent_fp8_kernel.argtypes = [vp, vp, vp, vp, vp, vp] + [i32] * 9 + [i64, i32, vp]
    lib.ggemm_persistent_fp8_kernel.restype = ctypes.c_int
    lib.ggemm_persistent_selected_kernel.argtypes = [i32] * 5
    lib.ggemm_persistent_selected_kernel.restype = ctypes.c_int32
    lib.ggemm_persistent_clear_tail.argtypes = [vp, i32, i32, vp, i32, i64, vp]
    lib.ggemm_persistent_clear_tail.restype = ctypes.c_int
    lib.ggemm_persistent_transpose_u8.argtypes = [vp, i32, i32, i32, i64, i64, vp, i64, i64, vp]
    lib.ggemm_persistent_transpose_u8.restype = ctypes.c_int
    lib.ggemm_quant_amax.argtypes = [vp, i32, i64, i32, i64, vp, vp]
    lib.ggemm_quant_amax.restype = ctypes.c_int
    lib.ggemm_quant_fp8_tensorwise.argtypes = [vp, i32, i64, i32, i64, i32, vp, i64, vp, vp, vp]
    lib.ggemm_quant_fp8_tensorwise.restype = ctypes.c_int
    lib.ggemm_quant_fp8_tensorwise_delayed.argtypes = [vp, i32, i64, i32, i64, i32, vp, i64, vp, i32, i32, vp, vp]
    lib.ggemm_quant_fp8_tensorwise_delayed.restype = ctypes.c_int
    lib.ggemm_quant_fp8_tensorwise_delayed_dev.argtypes = [vp, i32, i64, i32, i64, i32, vp, i64, vp, i32, vp, vp,
                                                           vp]
    lib.ggemm_quant_fp8_tensorwise_delayed_dev.restype = ctypes.c_int
    lib.ggemm_quant_fp8_tensorwise_transpose.argtypes = [vp, i32, i32, i32, i32, i32, vp, i64, vp, i64, vp, vp, vp]
    lib.ggemm_quant_fp8_tensorwise_transpose.restype = ctypes.c_int
    lib.ggemm_quant_fp8_tensorwise_transpose_delayed.argtypes = [vp, i32, i32, i32, i32, i32, vp, i64, vp, i64, vp,
                                                                 i32, i32, vp, vp]
    lib.ggemm_quant_fp8_tensorwise_transpose_delayed.restype = ctypes.c_int
    lib.ggemm_quant_fp8_tensorwise_transpose_delayed_dev.argtypes = [vp, i32, i32, i32, i32, i32, vp, i64, vp, i64,
                                                                     vp, i32, vp, vp, vp]
    lib.ggemm_quant_fp8_tensorwise_transpose_delayed_dev.restype = ctypes.c_int
    lib.ggemm_quant_mxfp8_grouped.argtypes = [vp, i32, i64, i32, i64, vp, i32, i32, vp, i64, i64, vp, i64, vp, vp]
    lib.ggemm_quant_mxfp8_grouped.restype = ctypes.c_int
    _lib = lib
    return lib


def strerror(code: int) -> str:
    try:
        return load().ggemm_vark_strerror(int(code)).decode()
    except Exception:  # library missing: still produce a message
        return ERRORS.get(code, "unknown")


def check(code: int, what: str) -> None:
    if code != 0:
        raise GGemmError(code, what)


def bf16_kernel(out_m: int, out_n: int, stride_cm: int | None = None) -> str:
    """Which kernel the bf16 wgrad entry points run for this shape (a 256-byte aligned C assumed):
    "wide320" / "wide256" (320 x 320 / 256 x 384 tiles, one wave per SIMD) or "192-row" (the
    reference launch geometry)."""
    sel = load().ggemm_vark_bf16_kernel(int(out_m), int(out_n), int(stride_cm or out_n), 256)
    return {320: "wide320", 256: "wide256"}.get(sel, "192-row")


def launch_geometry(out_n: int = 5760) -> dict:
    lib = load()
    vals = [ctypes.c_int32() for _ in range(5)]
    lib.ggemm_vark_launch_geometry(int(out_n), *[ctypes.byref(v) for v in vals])
    keys = ("block_threads", "dynamic_lds", "tile_m", "tile_n", "k_step")
    return {k: v.value for k, v in zip(keys, vals)}
