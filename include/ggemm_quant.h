/* C ABI of the MI355X FP8 quantization producer (libggemm_vark.so): the step before the grouped
 * GEMMs, which turns bf16 / fp32 activations, output gradients and weights into their fp8
 * operands and scales. Return codes, strerror and the ABI version are those of ggemm_vark.h.
 *
 * There is no counterpart inside the reference tree: its harness feeds the GEMMs with raw
 * randn -> fp8 casts and scales of 0.1 (reference bench.py:220-223,260-261) and leaves
 * quantization to the training framework (Primus-Turbo, not vendored). The recipes are the ones
 * the measured configurations define (per-tensor amax / fmax scales; e8m0 block exponents
 * floor(log2(block amax / fmax)) per 32 tokens, groups padded to multiples of 32 tokens).
 *
 * All pointers are device pointers; sizes and strides in elements. Launches are asynchronous on
 * `stream`; no allocation, no synchronization. Rounding: x / scale is the correctly rounded fp32
 * quotient; fp32 -> fp8 rounds to nearest even, subnormals included; values are clamped to
 * +-fmax first (448 for e4m3fn, 57344 for e5m2); NaN stays NaN (a NaN code, 0x7F or 0xFF: the
 * sign of a NaN is unspecified).
 */
#ifndef GGEMM_QUANT_H
#define GGEMM_QUANT_H

#include <stdint.h>

#include "ggemm_vark.h"

#ifdef __cplusplus
extern "C" {
#endif

/* input element types */
#define GGEMM_IN_BF16 0
#define GGEMM_IN_F32 1
/* output fp8 formats (same codes as ggemm_persistent.h) */
#ifndef GGEMM_FP8_E4M3
#define GGEMM_FP8_E4M3 0
#define GGEMM_FP8_E5M2 1
#endif

#define GGEMM_QUANT_MAX_GROUPS 2047

/* amax = max |x| over x [rows, cols] (row stride `stride`), written to amax_out (fp32). NaN
 * propagates. cols and stride multiples of 8, x 16-byte aligned. */
int ggemm_quant_amax(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride, float* amax_out,
                     void* stream);

/* Per-tensor quantization: amax_out = max |x|, scale_out = amax / fmax (1 when amax == 0),
 * out[r, c] = fp8(clamp(x[r, c] / scale, -fmax, fmax)). out: [rows, cols] bytes, row stride
 * out_stride (a multiple of 8), 8-byte aligned. A weight [G, N, K] is the 2-D [G*N, K]. The scale
 * is what ggemm_vark_wgrad_fp8 / ggemm_persistent_fp8 take as lhs_scale / rhs_scale / a_scale /
 * b_scale. */
int ggemm_quant_fp8_tensorwise(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride,
                               int32_t out_format, void* out, int64_t out_stride, float* scale_out,
                               float* amax_out, void* stream);

/* Longest amax history of ggemm_quant_fp8_tensorwise_delayed. */
#define GGEMM_QUANT_MAX_HISTORY 1024

/* Per-tensor quantization with delayed scaling: the scale comes from earlier amax values, and this
 * tensor's amax is recorded in the same pass (no separate amax pass over x). amax_history is a
 * device fp32 array of history_len entries; scale_out = m / fmax with m the largest entry other
 * than amax_history[slot] (1 when m == 0, NaN when an entry is NaN); out[r, c] = fp8(clamp(x[r, c]
 * / scale, -fmax, fmax)) with the same rounding as ggemm_quant_fp8_tensorwise; then
 * amax_history[slot] = max |x| of this x (NaN propagates). A caller cycling slot through the
 * history gets "the largest amax of the previous history_len - 1 calls" as its scale. Other
 * requirements as for ggemm_quant_fp8_tensorwise; 1 <= history_len <= GGEMM_QUANT_MAX_HISTORY,
 * 0 <= slot < history_len. No reference counterpart (the reference harness quantizes with fixed
 * scales, bench.py:220-223); the FP8 grouped linear layer's delayed-scaling recipe uses it. */
int ggemm_quant_fp8_tensorwise_delayed(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride,
                                       int32_t out_format, void* out, int64_t out_stride, float* amax_history,
                                       int32_t history_len, int32_t slot, float* scale_out, void* stream);

/* ggemm_quant_fp8_tensorwise_delayed with the slot kept on the device (ABI version 9): `slot` is a
 * device int32 holding the previous call's slot; the call first moves it to (slot + 1) mod
 * history_len (a value outside [0, history_len) restarts at 0) and clears that history entry, then
 * quantizes as ggemm_quant_fp8_tensorwise_delayed with it. The slot is read and advanced by the
 * launched kernels, so a HIP graph that captures the call rolls through the history on every
 * replay (with a host slot a replay would record into one fixed entry and scale by a frozen
 * history). A caller cycling slot 0, 1, ... through the host entry point gets the same results
 * from this one with *slot starting at history_len - 1. No reference counterpart. */
int ggemm_quant_fp8_tensorwise_delayed_dev(const void* x, int32_t in_dtype, int64_t rows, int32_t cols,
                                           int64_t stride, int32_t out_format, void* out, int64_t out_stride,
                                           float* amax_history, int32_t history_len, int32_t* slot,
                                           float* scale_out, void* stream);

/* Per-tensor quantization of a batch of matrices with a transposed copy: x is a contiguous
 * [batch, rows, cols] (a weight [G, N, K]); amax_out and scale_out as in
 * ggemm_quant_fp8_tensorwise over all batch*rows*cols elements;
 * out_t[(b * cols + c) * out_t_stride + r] = q[b, r, c] and, when out is not NULL,
 * out[(b * rows + r) * out_stride + c] = q[b, r, c]; q's bytes are exactly
 * ggemm_quant_fp8_tensorwise's. out_t is the data-gradient GEMM's K-major B (dx = dy @ w[g] reads
 * w[g]^T), so one pass over the weight feeds both the forward and the data-gradient GEMM. Row
 * strides (bytes) are multiples of 16, >= cols (out) and >= rows (out_t): a stride that is a
 * multiple of 128 keeps every row on whole cache lines, which the GEMMs read faster. rows and cols
 * multiples of 16; x, out and out_t 16-byte aligned. Padding bytes are not written. */
int ggemm_quant_fp8_tensorwise_transpose(const void* x, int32_t in_dtype, int32_t batch, int32_t rows, int32_t cols,
                                         int32_t out_format, void* out, int64_t out_stride, void* out_t,
                                         int64_t out_t_stride, float* scale_out, float* amax_out, void* stream);

/* The transposing pass with delayed scaling: out / out_t as in ggemm_quant_fp8_tensorwise_transpose,
 * the scale and amax_history as in ggemm_quant_fp8_tensorwise_delayed (the max |x| over all
 * batch*rows*cols elements recorded at amax_history[slot], no separate amax pass). No reference
 * counterpart; the FP8 grouped linear layer's delayed-scaling recipe quantizes its weight with it. */
int ggemm_quant_fp8_tensorwise_transpose_delayed(const void* x, int32_t in_dtype, int32_t batch, int32_t rows,
                                                 int32_t cols, int32_t out_format, void* out, int64_t out_stride,
                                                 void* out_t, int64_t out_t_stride, float* amax_history,
                                                 int32_t history_len, int32_t slot, float* scale_out, void* stream);

/* ggemm_quant_fp8_tensorwise_transpose_delayed with the slot kept on the device, advanced by the
 * call as in ggemm_quant_fp8_tensorwise_delayed_dev (ABI version 9). No reference counterpart. */
int ggemm_quant_fp8_tensorwise_transpose_delayed_dev(const void* x, int32_t in_dtype, int32_t batch, int32_t rows,
                                                     int32_t cols, int32_t out_format, void* out, int64_t out_stride,
                                                     void* out_t, int64_t out_t_stride, float* amax_history,
                                                     int32_t history_len, int32_t* slot, float* scale_out,
                                                     void* stream);

/* MX (OCP microscaling) quantization along the token axis with group-aligned padding, the input
 * of ggemm_vark_wgrad_mxfp8. x: [rows, cols] token-major; group_offs: int64 [G+1] (0-based,
 * non-decreasing, <= rows). Group g's rows are written to out rows padded_offs[g] ..
 * padded_offs[g] + len_g - 1, followed by zero rows up to the next multiple of 32; padded_offs
 * (int64 [G+1], written here) are the prefix sums of ceil(len/32)*32. Per 32-row block b and
 * column c: X = floor(log2(fl32(amax / fmax))) clamped to [-127, 127] (0 for an all-zero block,
 * the e8m0 NaN code 0xFF when the block holds a NaN), scales[b, c] = X + 127,
 * out[32b + i, c] = fp8(clamp(x * 2^-X, -fmax, fmax)). out: [out_rows, cols] bytes with
 * out_rows >= rows + 31*G, row stride a multiple of 16; scales: [out_rows / 32, cols] bytes, row
 * stride scale_stride (a multiple of 16). Rows past padded_offs[G] are not written. Offsets that
 * are decreasing or outside [0, rows] make the kernel write nothing. cols a multiple of 16. */
int ggemm_quant_mxfp8_grouped(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride,
                              const int64_t* group_offs, int32_t G, int32_t out_format, void* out,
                              int64_t out_stride, int64_t out_rows, uint8_t* scales, int64_t scale_stride,
                              int64_t* padded_offs, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GGEMM_QUANT_H */
