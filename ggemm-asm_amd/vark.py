"""PyTorch-facing grouped wgrad ops over the C ABI.

``grouped_gemm_fp8_tensorwise_variable_k`` mirrors the reference's oracle call
``grouped_gemm_fp8_tensorwise_variable_k_triton_kernel(lhs, rhs, lhs_scale, rhs_scale,
group_offs)`` (reference bench.py:241-246, 262-269): same argument order and meaning, a new
bf16 ``[G, OUT_M, OUT_N]`` tensor as the result. The launch goes through
``ggemm_vark_wgrad_fp8_out`` in libggemm_vark.so on torch's current stream, bounded by the
tensors' token count (group offsets past it are clamped on the device); there is no fallback: a
missing library or a non-gfx950 device raises.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

_FP8_LHS = (torch.float8_e4m3fn, torch.uint8)
_FP8_RHS = (torch.float8_e5m2, torch.uint8)


def _check_inputs(lhs, rhs, group_offs, lhs_dt=_FP8_LHS, rhs_dt=_FP8_RHS):
    if lhs.dim() != 2 or rhs.dim() != 2:
        raise ValueError("lhs and rhs must be 2-D [M_total, OUT_M] / [M_total, OUT_N]")
    if lhs.shape[0] != rhs.shape[0]:
        raise ValueError(f"token counts differ: lhs {tuple(lhs.shape)} vs rhs {tuple(rhs.shape)}")
    if lhs.dtype not in lhs_dt or rhs.dtype not in rhs_dt:
        raise TypeError(f"lhs must be float8_e4m3fn (or its uint8 bytes), rhs float8_e5m2; "
                        f"got {lhs.dtype}, {rhs.dtype}")
    if lhs.stride(1) != 1 or rhs.stride(1) != 1:
        raise ValueError("lhs/rhs must be contiguous along the feature dimension")
    for name, t in (("lhs", lhs), ("rhs", rhs)):
        # the kernels may read a token row up to its stride: the last row's padding must exist
        end = (t.storage_offset() + t.shape[0] * t.stride(0)) * t.element_size()
        if t.shape[0] > 0 and end > t.untyped_storage().nbytes():
            raise ValueError(f"{name}'s last row does not extend to its row stride ({t.stride(0)}) within its "
                             "storage: the kernels may read a row's padding; use a view into a tensor of full rows")
    if group_offs.dtype != torch.int64 or group_offs.dim() != 1 or group_offs.numel() < 2:
        raise ValueError("group_offs must be int64 [G+1]")
    dev = lhs.device
    for t in (rhs, group_offs):
        if t.device != dev:
            raise ValueError("all tensors must be on the same device")
    if dev.type != "cuda":
        raise ValueError("the variable-K wgrad runs on a gfx950 GPU only (tensors are on "
                         f"{dev}); use the CPU oracle in tests for reference results")


def _check_out(out, G, OUT_M, OUT_N, dev, dtype=torch.bfloat16):
    if out is None:
        return torch.empty((G, OUT_M, OUT_N), dtype=dtype, device=dev)
    if out.dtype != dtype or out.dim() != 3 or tuple(out.shape) != (G, OUT_M, OUT_N):
        raise ValueError(f"out must be {dtype} [{G}, {OUT_M}, {OUT_N}]")
    if out.device != dev:
        raise ValueError("out must be on the input device")
    return out


def _validate_offsets(group_offs, M_total, mx):
    offs = group_offs.detach().to("cpu", torch.int64).contiguous().numpy()
    G = offs.size - 1
    rc = _lib.load().ggemm_vark_check_offsets(
        offs.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), G, M_total, 1 if mx else 0)
    _lib.check(rc, "ggemm_vark_check_offsets")


def _nonempty(t: torch.Tensor) -> torch.Tensor:
    """A zero-token operand has a null data pointer; the kernel reads no row of it (every group is
    empty), so hand the library a one-row placeholder with the same width instead."""
    if t.shape[0] > 0:
        return t
    return torch.zeros((1, t.shape[1]), dtype=t.dtype, device=t.device)


def _stream(dev) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def grouped_gemm_fp8_tensorwise_variable_k(lhs: torch.Tensor, rhs: torch.Tensor, lhs_scale: torch.Tensor,
                                           rhs_scale: torch.Tensor, group_offs: torch.Tensor,
                                           out: torch.Tensor | None = None, *, mfma: str = "k128",
                                           validate: bool = False, out_dtype: torch.dtype = torch.bfloat16,
                                           accumulate: bool = False, wide: bool | int = False) -> torch.Tensor:
    """``out[g] = lhs_scale * rhs_scale * lhs[offs[g]:offs[g+1]]^T @ rhs[offs[g]:offs[g+1]]`` (bf16).

    lhs: float8_e4m3fn [M_total, OUT_M]; rhs: float8_e5m2 [M_total, OUT_N]; scales: fp32 scalar
    tensors on the device; group_offs: int64 [G+1]. ``mfma="k32"`` selects the kernel built on the
    K=32 MFMA the reference uses; ``validate=True`` checks group_offs on the host first (a sync).
    ``out_dtype=torch.float32`` writes an fp32 C; ``accumulate=True`` adds the result into the fp32
    ``out`` given (the main-grad accumulation, beta = 1). ``wide=True`` runs a wide-tile kernel
    (320 x 320 tiles where OUT_M and OUT_N are multiples of 320, else 256 x 384 with OUT_N a
    multiple of 384, bf16 C only); ``wide=320`` / ``wide=256`` picks the tile height. Without it the
    library picks (a wide tile for OUT_M >= 1024 where one fits).
    """
    _check_inputs(lhs, rhs, group_offs)
    for s in (lhs_scale, rhs_scale):
        if s.dtype != torch.float32 or s.numel() != 1 or s.device != lhs.device:
            raise ValueError("scales must be single-element fp32 tensors on the input device")
    G = group_offs.numel() - 1
    M_total, OUT_M = lhs.shape
    OUT_N = rhs.shape[1]
    if accumulate and out is None:
        raise ValueError("accumulate=True adds into an existing fp32 `out`")
    if accumulate:
        out_dtype = torch.float32
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("out_dtype must be torch.bfloat16 or torch.float32")
    out = _check_out(out, G, OUT_M, OUT_N, lhs.device, out_dtype)
    if validate:
        _validate_offsets(group_offs, M_total, mx=False)
    lhs, rhs = _nonempty(lhs), _nonempty(rhs)
    lib = _lib.load()
    if wide:
        if mfma != "k128":
            raise ValueError("the wide-tile kernels use the 32x32x64 MFMA (mfma='k128' family)")
        mode = 2 if accumulate else (1 if out_dtype == torch.float32 else 0)
        with torch.cuda.device(lhs.device):
            rc = lib.ggemm_vark_wgrad_fp8_wide(
                lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), lhs_scale.data_ptr(), rhs_scale.data_ptr(),
                group_offs.data_ptr(), G, OUT_M, OUT_N, lhs.stride(0), rhs.stride(0), out.stride(0), out.stride(1),
                out.stride(2), M_total, 0 if wide is True else int(wide), mode, _stream(lhs.device))
        _lib.check(rc, "ggemm_vark_wgrad_fp8_wide")
        return out
    if mfma == "k128":
        mode = 2 if accumulate else (1 if out_dtype == torch.float32 else 0)
        with torch.cuda.device(lhs.device):
            rc = lib.ggemm_vark_wgrad_fp8_out(
                lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), lhs_scale.data_ptr(), rhs_scale.data_ptr(),
                group_offs.data_ptr(), G, OUT_M, OUT_N, lhs.stride(0), rhs.stride(0), out.stride(0), out.stride(1),
                out.stride(2), mode, M_total, _stream(lhs.device))
        _lib.check(rc, "ggemm_vark_wgrad_fp8_out")
        return out
    if mfma != "k32":
        raise ValueError("mfma must be 'k128' or 'k32'")
    if out_dtype == torch.float32:
        raise ValueError("the fp32 output modes use the K=128 MFMA kernel")
    # the K=32 kernel keeps the reference's argument list (no token count): offsets must end
    # within the tensors, as with the reference kernel
    with torch.cuda.device(lhs.device):
        rc = lib.ggemm_vark_wgrad_fp8_k32(
            lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), lhs_scale.data_ptr(), rhs_scale.data_ptr(),
            group_offs.data_ptr(), G, OUT_M, OUT_N, lhs.stride(0), rhs.stride(0), out.stride(0), out.stride(1),
            out.stride(2), _stream(lhs.device))
    _lib.check(rc, "ggemm_vark_wgrad_fp8_k32")
    return out


def grouped_gemm_mxfp8_variable_k(lhs: torch.Tensor, rhs: torch.Tensor, lhs_scale: torch.Tensor,
                                  rhs_scale: torch.Tensor, group_offs: torch.Tensor,
                                  out: torch.Tensor | None = None, *, validate: bool = False,
                                  tile_m: int = 0) -> torch.Tensor:
    """MXFP8 variant: ``lhs_scale``/``rhs_scale`` are e8m0 bytes [ceil(M/32), OUT_M] / [.., OUT_N]
    (uint8 or float8_e8m0fnu); token block b of a column is scaled by 2^(scale-127). Group starts
    must be multiples of 32 (``validate=True`` checks it on the host). ``tile_m``: 0 lets the
    library pick (the 320 x 320 wide-tile kernel for OUT_M >= 1024 where both output dims are
    multiples of 320), 320 / 192 force the wide / the 192-row-tile kernel."""
    _check_inputs(lhs, rhs, group_offs)
    M_total, OUT_M = lhs.shape
    OUT_N = rhs.shape[1]
    nblk = (M_total + 31) // 32
    for s, w in ((lhs_scale, OUT_M), (rhs_scale, OUT_N)):
        if s.dtype not in (torch.uint8, getattr(torch, "float8_e8m0fnu", torch.uint8)):
            raise TypeError("MX scales must be e8m0 bytes (uint8 or float8_e8m0fnu)")
        if s.dim() != 2 or s.shape[0] < nblk or s.shape[1] != w or s.stride(1) != 1:
            raise ValueError(f"MX scales must be [{nblk}, width] with unit column stride")
        if s.device != lhs.device:
            raise ValueError("scales must be on the input device")
    G = group_offs.numel() - 1
    out = _check_out(out, G, OUT_M, OUT_N, lhs.device)
    if validate:
        _validate_offsets(group_offs, M_total, mx=True)
    lhs, rhs = _nonempty(lhs), _nonempty(rhs)
    lhs_scale, rhs_scale = _nonempty(lhs_scale), _nonempty(rhs_scale)
    lib = _lib.load()
    with torch.cuda.device(lhs.device):
        rc = lib.ggemm_vark_wgrad_mxfp8_tile(
            lhs.data_ptr(), rhs.data_ptr(), out.data_ptr(), lhs_scale.data_ptr(), rhs_scale.data_ptr(),
            group_offs.data_ptr(), G, OUT_M, OUT_N, lhs.stride(0), rhs.stride(0), out.stride(0), out.stride(1),
            out.stride(2), lhs_scale.stride(0), rhs_scale.stride(0), M_total, int(tile_m), _stream(lhs.device))
    _lib.check(rc, "ggemm_vark_wgrad_mxfp8_tile")
    return out


# --------------------------------------------------------------------------- torch.library op

def _register_custom_op():
    """``torch.ops.ggemm.variable_k_wgrad_fp8`` for callers that dispatch through torch."""
    try:
        lib_def = torch.library.Library("ggemm", "DEF")
    except Exception:  # already defined in this process
        return
    lib_def.define("variable_k_wgrad_fp8(Tensor lhs, Tensor rhs, Tensor lhs_scale, Tensor rhs_scale, "
                   "Tensor group_offs) -> Tensor")

    def _impl(lhs, rhs, lhs_scale, rhs_scale, group_offs):
        return grouped_gemm_fp8_tensorwise_variable_k(lhs, rhs, lhs_scale, rhs_scale, group_offs)

    def _meta(lhs, rhs, lhs_scale, rhs_scale, group_offs):
        return lhs.new_empty((group_offs.shape[0] - 1, lhs.shape[1], rhs.shape[1]), dtype=torch.bfloat16)

    lib_def.impl("variable_k_wgrad_fp8", _impl, "CUDA")
    lib_def.impl("variable_k_wgrad_fp8", _meta, "Meta")
    _register_custom_op.lib = lib_def  # keep the registration alive


_register_custom_op()


def as_bf16_bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> numpy uint16 bit patterns (host copy)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
