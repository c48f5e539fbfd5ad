"""CPU oracle for the FP8 quantization producer (per-tensor and MX with group padding).

TEST INFRASTRUCTURE ONLY. This module is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and never as the thing measured or shipped.

What it restates
----------------
The reference tree holds no quantizer: its harness casts ``torch.randn`` straight to fp8 and
passes scales of 0.1 (reference bench.py:220-223,260-261); quantization belongs to the training
framework (Primus-Turbo, not vendored). The recipes restated here are those of the measured
configurations:

* per-tensor: ``amax = max|x|``, ``scale = fl32(amax / fmax)`` (1 when amax == 0),
  ``q = fp8(clamp(fl32(x / scale), -fmax, fmax))``;
* per-tensor with delayed scaling (the layer's amax-history recipe; no reference counterpart):
  the same with amax taken as the largest entry of an amax history other than the slot this call
  replaces, and amax(x) recorded in that slot;
* MX along the token axis: per 32-token block and column ``X = floor(log2(fl32(amax / fmax)))``
  (exact floor of the fp32 quotient's log2) clamped to [-127, 127], 0 for an all-zero block,
  e8m0 byte ``X + 127``; ``q = fp8(clamp(x * 2^-X, -fmax, fmax))``; each group padded with zero rows
  to a multiple of 32, padded offsets the prefix sums of ``ceil(len/32) * 32``.

``fp8()`` rounds to nearest even (subnormals included); NaN maps to a NaN code, ``0x7F | sign``
here (the sign of a NaN result is unspecified in IEEE arithmetic, and e5m2 has three NaN codes,
0x7D-0x7F, so checks compare NaN-ness).

Pinning (tests/test_oracle_quant.py): the encoder against torch's own float8 casts on every fp8
value, every midpoint between neighbours (ties), both neighbours of each midpoint and random fp32
values over the whole range; the per-tensor and MX recipes against their torch restatements in
``ggemm_asm_amd.inputs`` on random data; the MX exponent rule against exact rational arithmetic
at and around powers of two; the padded layout against quantizing zero-padded groups one by one;
the delayed recipe against torch (scale from the history by torch's max and division, bytes by
torch's float8 cast of the clamped quotient), the slot's old entry ignored, saturation codes and
the special histories (all zero, NaN).
"""
from __future__ import annotations

import numpy as np

FMAX = {"e4m3": np.float32(448.0), "e5m2": np.float32(57344.0)}


def encode_fp8(x, fmt: str) -> np.ndarray:
    """fp32 -> fp8 bytes, round to nearest even. Values beyond +-fmax must be clamped first
    (they are not saturated here); NaN -> 0x7F | sign."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    s = ((u >> 24) & 0x80).astype(np.uint8)
    a = u & 0x7FFFFFFF
    if fmt == "e4m3":
        mant, min_normal, rebias, sub_mul = 3, 0x3C800000, (127 - 7) << 3, np.float32(512.0)
    elif fmt == "e5m2":
        mant, min_normal, rebias, sub_mul = 2, 0x38800000, (127 - 15) << 2, np.float32(65536.0)
    else:
        raise ValueError(fmt)
    shift = 23 - mant
    normal = (a + ((1 << (shift - 1)) - 1) + ((a >> shift) & 1)) >> shift
    normal = (normal - rebias) & 0xFF
    with np.errstate(invalid="ignore"):
        sub = np.nan_to_num(np.rint(np.abs(x) * sub_mul)).astype(np.uint64) & 0xFF
    out = np.where(a >= min_normal, normal, sub).astype(np.uint8)
    out = np.where(a > 0x7F800000, np.uint8(0x7F), out)
    return out | s


def _clamp(v: np.ndarray, fmt: str) -> np.ndarray:
    m = FMAX[fmt]
    return np.where(np.isnan(v), v, np.minimum(np.maximum(v, -m), m)).astype(np.float32)


def amax(x) -> np.float32:
    x = np.asarray(x, dtype=np.float32)
    return np.float32(np.max(np.abs(x))) if x.size else np.float32(0.0)   # np.max propagates NaN


def tensor_scale(am, fmt: str) -> np.float32:
    """fl32(amax / fmax); 1 for amax == 0; NaN stays NaN."""
    am = np.float32(am)
    if am > 0:
        return np.float32(am / FMAX[fmt])
    return np.float32(1.0) if am == 0 else am


def quantize_with_scale(x, scale, fmt: str) -> np.ndarray:
    """fp8(clamp(fl32(x / scale), -fmax, fmax)) bytes for a given fp32 scale."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        return encode_fp8(_clamp((x / np.float32(scale)).astype(np.float32), fmt), fmt)


def quantize_tensorwise(x, fmt: str):
    """(q bytes, scale, amax) of the per-tensor recipe; x float32 (bf16 inputs widened exactly)."""
    x = np.asarray(x, dtype=np.float32)
    am = amax(x)
    scale = tensor_scale(am, fmt)
    return quantize_with_scale(x, scale, fmt), scale, am


def quantize_tensorwise_delayed(x, history, slot: int, fmt: str):
    """Delayed scaling: (q bytes, scale, new history). The scale is tensor_scale of the largest
    |entry| of the amax history other than ``slot`` (NaN when one is NaN); x quantizes with it
    (values beyond fmax * scale saturate); the new history holds amax(x) at ``slot``."""
    x = np.asarray(x, dtype=np.float32)
    h = np.asarray(history, dtype=np.float32).copy()
    others = np.abs(np.delete(h, slot))
    m = np.float32(np.max(others)) if others.size else np.float32(0.0)   # np.max propagates NaN
    scale = tensor_scale(m, fmt)
    h[slot] = amax(x)
    return quantize_with_scale(x, scale, fmt), scale, h


def block_exponent(amax_blk, fmt: str) -> np.ndarray:
    """X = floor(log2(fl32(amax / fmax))) clamped to [-127, 127]; 0 for 0; 128 (byte 0xFF) for NaN."""
    a = np.asarray(amax_blk, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        y = (a / FMAX[fmt]).astype(np.float32)
        _, e = np.frexp(y)                          # y = m 2^e, m in [0.5, 1): floor(log2 y) = e - 1
    X = np.clip(e.astype(np.int64) - 1, -127, 127)
    X = np.where(np.isinf(y), 127, X)
    X = np.where(a == 0, 0, X)
    X = np.where(np.isnan(a), 128, X)
    return X


def padded_offsets(group_offs) -> np.ndarray:
    offs = np.asarray(group_offs, dtype=np.int64)
    lens = np.diff(offs)
    return np.concatenate([[0], np.cumsum((lens + 31) // 32 * 32)]).astype(np.int64)


def quantize_mx_grouped(x, group_offs, fmt: str, out_rows: int | None = None):
    """(q [out_rows, N] bytes, scales [out_rows/32, N] bytes, padded_offs [G+1]) of the MX recipe
    with group padding; rows past padded_offs[G] are left 0 here (the kernel leaves them unwritten)."""
    x = np.asarray(x, dtype=np.float32)
    offs = np.asarray(group_offs, dtype=np.int64)
    pad = padded_offsets(offs)
    M, N = x.shape
    G = offs.size - 1
    rows = out_rows if out_rows is not None else (M + 31 * G + 31) // 32 * 32
    xp = np.zeros((rows, N), dtype=np.float32)
    for g in range(G):
        lo, hi = int(offs[g]), int(offs[g + 1])
        xp[pad[g]:pad[g] + hi - lo] = x[lo:hi]
    nb = int(pad[-1]) // 32
    q = np.zeros((rows, N), dtype=np.uint8)
    scales = np.zeros((rows // 32, N), dtype=np.uint8)
    if nb:
        blk = xp[:32 * nb].reshape(nb, 32, N)
        am = np.max(np.abs(blk), axis=1)
        X = block_exponent(am, fmt)
        scales[:nb] = (X + 127).astype(np.uint8)
        mul = np.where(X == 128, np.float32(np.nan), np.ldexp(np.float32(1.0), -np.minimum(X, 127))).astype(np.float32)
        with np.errstate(invalid="ignore", over="ignore", under="ignore"):
            v = (blk * mul[:, None, :]).astype(np.float32)
        q[:32 * nb] = encode_fp8(_clamp(v, fmt), fmt).reshape(32 * nb, N)
    return q, scales, pad
