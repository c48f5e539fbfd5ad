"""PyTorch-facing FP8 quantization producer over the C ABI (include/ggemm_quant.h).

The step before the grouped GEMMs: per-tensor quantization (amax, scale = amax / fmax, saturating
round-to-nearest-even cast) for the tensorwise kernels, and MX quantization along the token axis
with group-aligned padding (e8m0 exponents per 32-token block and column) for the MXFP8 wgrad.
The reference tree holds no quantizer (its harness casts randn straight to fp8 with scales of 0.1,
reference bench.py:220-223,260-261); the recipes are those of the measured configurations. Every
launch goes through libggemm_vark.so on torch's current stream; there is no CPU path.
"""
from __future__ import annotations

import torch

from . import _lib
from .vark import _stream

GGEMM_IN_BF16 = 0
GGEMM_IN_F32 = 1
_IN = {torch.bfloat16: GGEMM_IN_BF16, torch.float32: GGEMM_IN_F32}
_OUT = {"e4m3": (0, torch.float8_e4m3fn), "e5m2": (1, torch.float8_e5m2)}
MAX_GROUPS = 2047


def _as_2d(x: torch.Tensor) -> torch.Tensor:
    if x.dim() < 2:
        raise ValueError("x must have at least 2 dimensions (rows x cols)")
    if x.dim() > 2:
        if not x.is_contiguous():
            raise ValueError("an N-d input must be contiguous (it is read as [prod(leading dims), last dim])")
        x = x.reshape(-1, x.shape[-1])
    if x.stride(1) != 1:
        raise ValueError("x must be contiguous along its last dimension")
    if x.shape[0] > 1 and x.stride(0) < x.shape[1]:
        # overlapping rows (an expanded or otherwise aliased view): the kernels read rows * cols
        # distinct elements, so hand them a copy that holds them
        x = x.contiguous()
    return x


def _row_stride(x2: torch.Tensor) -> int:
    """Row stride to hand the library for a 2-D view from ``_as_2d``: its own, except for a view of
    at most one row, whose stride(0) torch leaves arbitrary and the kernels never use."""
    return x2.stride(0) if x2.shape[0] > 1 else x2.shape[1]


def _ptr(x2: torch.Tensor) -> int:
    """A zero-row input has a null data pointer; the kernels read no row of it, so the library
    gets a one-row placeholder of the same width (and rows = 0)."""
    if x2.shape[0] > 0:
        return x2.data_ptr()
    _ptr.keep = torch.empty((1, x2.shape[1]), dtype=x2.dtype, device=x2.device)
    return _ptr.keep.data_ptr()


def _check(x: torch.Tensor, fmt: str):
    if x.dtype not in _IN:
        raise TypeError(f"x must be bfloat16 or float32, got {x.dtype}")
    if fmt not in _OUT:
        raise ValueError(f"fmt must be 'e4m3' or 'e5m2', got {fmt!r}")
    if x.device.type != "cuda":
        raise ValueError(f"the quantizer runs on a gfx950 GPU only (x is on {x.device}); use the CPU "
                         "oracle in tests for reference results")


def amax(x: torch.Tensor) -> torch.Tensor:
    """max |x| as a single-element fp32 tensor on x's device (NaN propagates)."""
    _check(x, "e4m3")
    x2 = _as_2d(x)
    out = torch.empty((), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = _lib.load().ggemm_quant_amax(_ptr(x2), _IN[x.dtype], x2.shape[0], x2.shape[1], _row_stride(x2),
                                          out.data_ptr(), _stream(x.device))
    _lib.check(rc, "ggemm_quant_amax")
    return out


def _padded_empty(shape, row_align, dt, device):
    """An fp8 tensor of `shape` whose rows start on multiples of `row_align` bytes (a view of a
    buffer with padded rows; None = contiguous)."""
    last = shape[-1]
    if not row_align or last % row_align == 0:
        return torch.empty(shape, dtype=dt, device=device)
    if row_align % 16:
        raise ValueError("row_align must be a multiple of 16 bytes")
    padded = (last + row_align - 1) // row_align * row_align
    return torch.empty(tuple(shape[:-1]) + (padded,), dtype=dt, device=device)[..., :last]


def quantize_fp8_tensorwise(x: torch.Tensor, fmt: str = "e4m3", row_align: int | None = None):
    """Per-tensor FP8 quantization. Returns ``(q, scale, amax)``: q has x's shape and dtype
    float8_e4m3fn / float8_e5m2, ``scale = amax / fmax`` (1 when amax == 0) and ``amax`` are
    single-element fp32 device tensors; ``q * scale`` dequantizes. The GEMM entry points take
    ``scale`` as their per-tensor scale. ``row_align=128`` returns q as a view whose rows start on
    128-byte lines (a padded buffer; the padding is not written): the persistent GEMM reads such
    operands with one cache line per row segment instead of 1.5 (K = 2880: 6-9% faster)."""
    _check(x, fmt)
    x2 = _as_2d(x)
    code, dt = _OUT[fmt]
    q = _padded_empty(x.shape, row_align, dt, x.device)
    # q's rows, contiguous or padded, are evenly strided over one buffer
    q2 = q.as_strided((x2.shape[0], x.shape[-1]), (q.stride(-2), 1))
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    am = torch.empty((), dtype=torch.float32, device=x.device)
    qp = q2 if q2.shape[0] > 0 else torch.empty((1, x.shape[-1]), dtype=dt, device=x.device)
    with torch.cuda.device(x.device):
        rc = _lib.load().ggemm_quant_fp8_tensorwise(
            _ptr(x2), _IN[x.dtype], x2.shape[0], x2.shape[1], _row_stride(x2), code, qp.data_ptr(),
            _row_stride(qp), scale.data_ptr(), am.data_ptr(), _stream(x.device))
    _lib.check(rc, "ggemm_quant_fp8_tensorwise")
    return q, scale, am


def quantize_fp8_tensorwise_delayed(x: torch.Tensor, amax_history: torch.Tensor, slot, fmt: str = "e4m3",
                                    row_align: int | None = None):
    """Per-tensor FP8 quantization with delayed scaling. ``amax_history``: fp32 [H] on x's device;
    the scale is ``max(amax_history[i] for i != slot) / fmax`` (1 when those are all 0), computed on
    the device, and ``amax_history[slot]`` becomes this x's amax in the same pass (no separate amax
    pass). Returns ``(q, scale)`` as ``quantize_fp8_tensorwise`` does; values beyond ``fmax * scale``
    saturate to +-fmax.

    ``slot``: an int in [0, H), or a one-element int32 tensor on x's device holding the previous
    call's slot, which the call advances to ``(slot + 1) % H`` on the device before using it -- the
    form a HIP graph capture replays correctly (each replay moves on through the history)."""
    _check(x, fmt)
    _check_history(amax_history, slot, x.device)
    H = amax_history.numel()
    dev_slot = isinstance(slot, torch.Tensor)
    x2 = _as_2d(x)
    code, dt = _OUT[fmt]
    q = _padded_empty(x.shape, row_align, dt, x.device)
    q2 = q.as_strided((x2.shape[0], x.shape[-1]), (q.stride(-2), 1))
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    qp = q2 if q2.shape[0] > 0 else torch.empty((1, x.shape[-1]), dtype=dt, device=x.device)
    name = "ggemm_quant_fp8_tensorwise_delayed" + ("_dev" if dev_slot else "")
    with torch.cuda.device(x.device):
        rc = getattr(_lib.load(), name)(
            _ptr(x2), _IN[x.dtype], x2.shape[0], x2.shape[1], _row_stride(x2), code, qp.data_ptr(),
            _row_stride(qp), amax_history.data_ptr(), H, slot.data_ptr() if dev_slot else slot, scale.data_ptr(),
            _stream(x.device))
    _lib.check(rc, name)
    return q, scale


def quantize_fp8_tensorwise_transpose(x: torch.Tensor, fmt: str = "e4m3", keep: bool = True,
                                      row_align: int | None = None):
    """Per-tensor FP8 quantization of a contiguous [B, R, C] (or [R, C]) tensor with a transposed
    copy, in one pass. Returns ``(q, q_t, scale, amax)``: ``q`` is ``quantize_fp8_tensorwise(x)``'s
    q (None when ``keep`` is False), ``q_t`` the [B, C, R] (or [C, R]) transpose of the same bytes.
    For a weight [G, N, K], ``q`` is the forward GEMM's B and ``q_t`` the data-gradient GEMM's
    (``dy @ w[g]`` reads ``w[g]^T`` K-major). ``row_align`` as in ``quantize_fp8_tensorwise``, for
    both outputs. R and C must be multiples of 16."""
    return _transpose(x, fmt, keep, row_align, None, 0)


def quantize_fp8_tensorwise_transpose_delayed(x: torch.Tensor, amax_history: torch.Tensor, slot,
                                              fmt: str = "e4m3", keep: bool = True, row_align: int | None = None):
    """``quantize_fp8_tensorwise_transpose`` with delayed scaling: the scale from ``amax_history``'s
    entries other than ``slot`` and x's amax recorded at ``slot`` in the same pass, as in
    ``quantize_fp8_tensorwise_delayed`` (``slot`` an int, or a device int32 tensor the call
    advances). Returns ``(q, q_t, scale)``."""
    q, q_t, scale, _ = _transpose(x, fmt, keep, row_align, amax_history, slot)
    return q, q_t, scale


def _check_history(amax_history: torch.Tensor, slot, device):
    if amax_history.dtype != torch.float32 or amax_history.dim() != 1 or not amax_history.is_contiguous():
        raise ValueError("amax_history must be a contiguous fp32 [H] tensor")
    if amax_history.device != device:
        raise ValueError("amax_history must be on x's device")
    if isinstance(slot, torch.Tensor):
        if slot.dtype != torch.int32 or slot.numel() != 1 or slot.device != device:
            raise ValueError("a device slot must be a one-element int32 tensor on x's device")
    elif not 0 <= slot < amax_history.numel():
        raise ValueError(f"slot {slot} outside the history of {amax_history.numel()}")


def _transpose(x, fmt, keep, row_align, amax_history, slot):
    _check(x, fmt)
    if x.dim() not in (2, 3) or not x.is_contiguous():
        raise ValueError("x must be a contiguous [B, R, C] or [R, C] tensor")
    if amax_history is not None:
        _check_history(amax_history, slot, x.device)
    x3 = x if x.dim() == 3 else x.unsqueeze(0)
    B, R, C = x3.shape
    if R % 16 or C % 16:
        raise ValueError(f"R and C must be multiples of 16, got {R} x {C}")
    code, dt = _OUT[fmt]
    q = _padded_empty(x.shape, row_align, dt, x.device) if keep else None
    q_t = _padded_empty(x.shape[:-2] + (C, R), row_align, dt, x.device)
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    q_stride = q.stride(-2) if keep else C
    t_stride = q_t.stride(-2)
    if B == 0:                                   # nothing to read: a one-matrix placeholder pointer
        xp = torch.empty((R, C), dtype=x.dtype, device=x.device).data_ptr()
        tp = torch.empty((C, t_stride), dtype=dt, device=x.device).data_ptr()
        qp = torch.empty((R, q_stride), dtype=dt, device=x.device).data_ptr() if keep else None
    else:
        xp, tp, qp = x.data_ptr(), q_t.data_ptr(), (q.data_ptr() if keep else None)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        if amax_history is None:
            am = torch.empty((), dtype=torch.float32, device=x.device)
            name = "ggemm_quant_fp8_tensorwise_transpose"
            rc = lib.ggemm_quant_fp8_tensorwise_transpose(
                xp, _IN[x.dtype], B, R, C, code, qp, q_stride, tp, t_stride, scale.data_ptr(), am.data_ptr(),
                _stream(x.device))
        else:
            am = None
            dev_slot = isinstance(slot, torch.Tensor)
            name = "ggemm_quant_fp8_tensorwise_transpose_delayed" + ("_dev" if dev_slot else "")
            rc = getattr(lib, name)(
                xp, _IN[x.dtype], B, R, C, code, qp, q_stride, tp, t_stride, amax_history.data_ptr(),
                amax_history.numel(), slot.data_ptr() if dev_slot else slot, scale.data_ptr(), _stream(x.device))
    _lib.check(rc, name)
    return q, q_t, scale, am


def padded_rows(rows: int, G: int) -> int:
    """Output rows that ``quantize_mxfp8_grouped`` needs: every group padded to 32 rows fits."""
    return (rows + 31 * G + 31) // 32 * 32


def quantize_mxfp8_grouped(x: torch.Tensor, group_offs: torch.Tensor, fmt: str = "e4m3"):
    """MX quantization along the token axis (rows) with group-aligned padding.

    x: bfloat16 / float32 [M, N] token-major; group_offs: int64 [G+1] on the device. Returns
    ``(q, scales, padded_offs)``: q fp8 [padded_rows(M, G), N] (group g at rows padded_offs[g] ..,
    zero rows up to the next multiple of 32; rows past padded_offs[G] are unspecified), scales
    uint8 e8m0 [padded_rows / 32, N], padded_offs int64 [G+1]. The three are the MX wgrad's inputs
    (with the matching tensor of the other operand, padded with the same offsets)."""
    _check(x, fmt)
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be 2-D [M, N], contiguous along N")
    x = _as_2d(x)
    if group_offs.dtype != torch.int64 or group_offs.dim() != 1 or group_offs.numel() < 2:
        raise ValueError("group_offs must be int64 [G+1]")
    if group_offs.device != x.device:
        raise ValueError("group_offs must be on x's device")
    M, N = x.shape
    G = group_offs.numel() - 1
    rows_out = padded_rows(M, G)
    code, dt = _OUT[fmt]
    q = torch.empty((rows_out, N), dtype=dt, device=x.device)
    scales = torch.empty((rows_out // 32, N), dtype=torch.uint8, device=x.device)
    padded = torch.empty(G + 1, dtype=torch.int64, device=x.device)
    with torch.cuda.device(x.device):
        rc = _lib.load().ggemm_quant_mxfp8_grouped(
            _ptr(x), _IN[x.dtype], M, N, _row_stride(x), group_offs.data_ptr(), G, code, q.data_ptr(),
            q.stride(0), rows_out, scales.data_ptr(), scales.stride(0), padded.data_ptr(), _stream(x.device))
    _lib.check(rc, "ggemm_quant_mxfp8_grouped")
    return q, scales, padded
