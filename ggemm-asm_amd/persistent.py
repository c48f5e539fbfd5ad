"""PyTorch-facing persistent grouped FP8 GEMM (forward / data-gradient sites) over the C ABI.

``grouped_gemm_fp8_tensorwise`` mirrors the reference's oracle call
``grouped_gemm_fp8_tensorwise_triton_kernel(a, b, a_scale, b_scale, group_offs, trans_b=...)``
(reference bench.py:238-247, call sites bench.py:153-180): same argument order and meaning, a new
bf16 ``[M_total, N]`` tensor as the result. The launch goes through ``ggemm_persistent_fp8`` in
libggemm_vark.so (include/ggemm_persistent.h) on torch's current stream; there is no fallback: a
missing library or a non-gfx950 device raises.
"""
from __future__ import annotations

import torch

from . import _lib
from .vark import _stream, _validate_offsets

GGEMM_FP8_E4M3 = 0
GGEMM_FP8_E5M2 = 1
MAX_GROUPS = 2047

_FORMATS = {torch.float8_e4m3fn: GGEMM_FP8_E4M3, torch.float8_e5m2: GGEMM_FP8_E5M2}
_FORMAT_NAMES = {"e4m3": GGEMM_FP8_E4M3, "e5m2": GGEMM_FP8_E5M2}


# kernel choices of ggemm_persistent_fp8_kernel (include/ggemm_persistent.h)
KERNELS = {"auto": 0, "512": 1, "wide": 2}


def selected_kernel(N: int, K: int, stride_am: int, stride_bn: int, stride_cm: int) -> str:
    """The kernel the library runs for this shape and these strides ("512" or "wide")."""
    k = _lib.load().ggemm_persistent_selected_kernel(N, K, stride_am, stride_bn, stride_cm)
    return {v: n for n, v in KERNELS.items()}[k]


def _a_format(a: torch.Tensor, a_format: str | None) -> int:
    if a_format is not None:
        if a_format not in _FORMAT_NAMES:
            raise ValueError(f"a_format must be 'e4m3' or 'e5m2', got {a_format!r}")
        fmt = _FORMAT_NAMES[a_format]
        if a.dtype in _FORMATS and _FORMATS[a.dtype] != fmt:
            raise TypeError(f"a_format={a_format!r} contradicts a.dtype={a.dtype}")
        if a.dtype not in _FORMATS and a.dtype != torch.uint8:
            raise TypeError(f"a must hold fp8 bytes, got {a.dtype}")
        return fmt
    if a.dtype not in _FORMATS:
        raise TypeError(f"a must be float8_e4m3fn or float8_e5m2 (or uint8 bytes with a_format=...); "
                        f"got {a.dtype}")
    return _FORMATS[a.dtype]


def transpose_b(b: torch.Tensor) -> torch.Tensor:
    """[G, K, N] fp8 (N contiguous) -> a new contiguous [G, N, K] tensor of the same bytes, through
    ``ggemm_persistent_transpose_u8`` (K and N multiples of 16)."""
    if b.dim() != 3 or b.stride(2) != 1:
        raise ValueError("b must be a 3-D [G, K, N] tensor contiguous along N")
    G, K, N = b.shape
    if b.device.type != "cuda":
        raise ValueError(f"the byte transpose runs on a gfx950 GPU only (b is on {b.device})")
    out = torch.empty((G, N, K), dtype=b.dtype, device=b.device)
    if G == 0 or K == 0 or N == 0:
        return out
    with torch.cuda.device(b.device):
        rc = _lib.load().ggemm_persistent_transpose_u8(b.data_ptr(), G, K, N, b.stride(0), b.stride(1), out.data_ptr(),
                                                       out.stride(0), out.stride(1), _stream(b.device))
    _lib.check(rc, "ggemm_persistent_transpose_u8")
    return out


def grouped_gemm_fp8_tensorwise(a: torch.Tensor, b: torch.Tensor, a_scale: torch.Tensor, b_scale: torch.Tensor,
                                group_offs: torch.Tensor, trans_b: bool = True, out: torch.Tensor | None = None,
                                *, a_format: str | None = None, validate: bool = False,
                                zero_tail: bool = False, kernel: str = "auto") -> torch.Tensor:
    """``out[r] = a_scale * b_scale * a[r] @ B[g]^T`` for ``offs[g] <= r < offs[g+1]`` (bf16).

    a: float8_e4m3fn (forward) or float8_e5m2 (data gradient) [M_total, K]; b: float8_e4m3fn
    [G, N, K] (``trans_b=True``, the layout of every reference call site) or [G, K, N]
    (``trans_b=False``: transposed into a contiguous [G, N, K] copy first by the library's byte
    transpose -- a weight quantized with ``quantize_fp8_tensorwise_transpose`` already has that
    layout); scales: single-element
    fp32 tensors on the device; group_offs: int64 [G+1]. Rows outside ``[0, offs[G])`` of ``out``
    are left unwritten, or set to zero with ``zero_tail=True`` (the library's device-side clear, no
    sync: dropped tokens get exact zeros). ``validate=True`` checks group_offs on the host first (a
    sync). Offsets past M_total are clamped to it on the device. ``kernel``: "auto" (the library's
    choice: the wide-tile kernel where N % 320 == 0 and K % 64 == 0, else the 512-thread kernel),
    "512" or "wide" (GGemmError GGEMM_E_SHAPE where the wide kernel does not apply).
    """
    if a.dim() != 2 or b.dim() != 3:
        raise ValueError("a must be 2-D [M_total, K] and b 3-D [G, N, K] (trans_b) or [G, K, N]")
    fmt = _a_format(a, a_format)
    if b.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"b must be float8_e4m3fn (or its uint8 bytes), got {b.dtype}")
    if group_offs.dtype != torch.int64 or group_offs.dim() != 1 or group_offs.numel() < 2:
        raise ValueError("group_offs must be int64 [G+1]")
    G = group_offs.numel() - 1
    if b.shape[0] != G:
        raise ValueError(f"b holds {b.shape[0]} groups, group_offs {G}")
    dev = a.device
    for t in (b, group_offs, a_scale, b_scale):
        if t.device != dev:
            raise ValueError("all tensors must be on the same device")
    if dev.type != "cuda":
        raise ValueError("the persistent grouped GEMM runs on a gfx950 GPU only (tensors are on "
                         f"{dev}); use the CPU oracle in tests for reference results")
    for s in (a_scale, b_scale):
        if s.dtype != torch.float32 or s.numel() != 1:
            raise ValueError("scales must be single-element fp32 tensors")
    if not trans_b:
        b = transpose_b(b)
    M_total, K = a.shape
    N = b.shape[1]
    if b.shape[2] != K:
        raise ValueError(f"K of a ({K}) and b ({b.shape[2]}) differ")
    if a.stride(1) != 1 or b.stride(2) != 1:
        raise ValueError("a and b must be contiguous along K")
    if out is None:
        out = torch.empty((M_total, N), dtype=torch.bfloat16, device=dev)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (M_total, N) or out.device != dev:
        raise ValueError(f"out must be bf16 [{M_total}, {N}] on the input device")
    if validate:
        _validate_offsets(group_offs, M_total, mx=False)
    if kernel not in KERNELS:
        raise ValueError(f"kernel must be one of {sorted(KERNELS)}, got {kernel!r}")
    if M_total == 0:
        return out
    lib = _lib.load()
    with torch.cuda.device(dev):
        rc = lib.ggemm_persistent_fp8_kernel(
            a.data_ptr(), b.data_ptr(), out.data_ptr(), a_scale.data_ptr(), b_scale.data_ptr(), group_offs.data_ptr(),
            G, N, K, a.stride(0), b.stride(0), b.stride(1), out.stride(0), out.stride(1), fmt, M_total,
            KERNELS[kernel], _stream(dev))
        _lib.check(rc, "ggemm_persistent_fp8_kernel")
        if zero_tail:
            rc = lib.ggemm_persistent_clear_tail(out.data_ptr(), N, out.stride(0), group_offs.data_ptr(), G, M_total,
                                                 _stream(dev))
            _lib.check(rc, "ggemm_persistent_clear_tail")
    return out


def _register_custom_op():
    """``torch.ops.ggemm_persistent.grouped_fp8`` for callers that dispatch through torch."""
    try:
        lib_def = torch.library.Library("ggemm_persistent", "DEF")
    except Exception:  # already defined in this process
        return
    lib_def.define("grouped_fp8(Tensor a, Tensor b, Tensor a_scale, Tensor b_scale, Tensor group_offs, "
                   "bool trans_b=True) -> Tensor")

    def _impl(a, b, a_scale, b_scale, group_offs, trans_b=True):
        return grouped_gemm_fp8_tensorwise(a, b, a_scale, b_scale, group_offs, trans_b)

    def _meta(a, b, a_scale, b_scale, group_offs, trans_b=True):
        return a.new_empty((a.shape[0], b.shape[1] if trans_b else b.shape[2]), dtype=torch.bfloat16)

    lib_def.impl("grouped_fp8", _impl, "CUDA")
    lib_def.impl("grouped_fp8", _meta, "Meta")
    _register_custom_op.lib = lib_def  # keep the registration alive


_register_custom_op()
