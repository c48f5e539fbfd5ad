/* C ABI of the MI355X persistent grouped FP8 GEMM (forward and data-gradient sites), exported by
 * libggemm_vark.so next to the variable-K entry points of ggemm_vark.h (return codes, strerror
 * and ABI version are shared).
 *
 *   out[r, :] = a_scale * b_scale * A[r, :] @ B[g]^T      for offs[g] <= r < offs[g+1]
 *
 * All pointers are device pointers; sizes and strides are in elements. Returns 0 on success, a
 * positive hipError_t value when the HIP runtime failed, or a negative GGEMM_E_* code when
 * argument validation failed (nothing is launched then). Launches are asynchronous on `stream`
 * (a hipStream_t; NULL = the null stream). No allocation, no state between calls, no sync.
 */
#ifndef GGEMM_PERSISTENT_H
#define GGEMM_PERSISTENT_H

#include <stdint.h>

#include "ggemm_vark.h"

#ifdef __cplusplus
extern "C" {
#endif

/* fp8 format codes of the A operand */
#define GGEMM_FP8_E4M3 0   /* float8_e4m3fn: forward sites (x, swiglu output) */
#define GGEMM_FP8_E5M2 1   /* float8_e5m2: data-gradient sites (output gradients) */

/* Largest G: the group offsets and per-group tile prefix sums live in on-chip memory. */
#define GGEMM_PERSISTENT_MAX_GROUPS 2047

/* Grouped FP8 GEMM with a per-group weight, trans_b layout. Replaces the reference's code-object
 * launch of `_grouped_fp8_persistent_gemm_kernel` (reference bench.py:312-361
 * prepare_persistent_args / launch_persistent_kernel: the same 14 data arguments in the same
 * order) and the Triton op it stands in for (reference bench.py:238-247,
 * `_triton_fwd(a, b, a_scale, b_scale, group_offs, trans_b=True)`), at the call sites of
 * reference bench.py:153-180 (gate_up_fwd, down_fwd, down_dgrad, gate_up_dgrad).
 *   a:   fp8 [M_total, K] in format a_format, row stride stride_am;
 *   b:   float8_e4m3fn [G, N, K], strides stride_bg, stride_bn (K contiguous);
 *   out: bf16 [M_total, N], strides stride_cm, stride_cn == 1;
 *   a_scale / b_scale: fp32 scalars; group_offs: int64 [G+1], offs[0] = 0, non-decreasing,
 *   offs[G] <= M_total. Rows of out outside [0, offs[G]) are not written.
 * M_total (rows of a and out) is not part of the reference kernarg; it bounds the 32-bit row and
 * tile indices here (M_total < 2^31 - 256, at most 2^30 output tiles of 192 x 320), and the
 * kernel clamps every group offset to M_total on the device, so offsets past it read and write no
 * row outside a and out (group g covers rows [min(offs[g], M_total), min(offs[g+1], M_total)));
 * a negative or decreasing offset array writes nothing.
 * Requirements: 1 <= G <= GGEMM_PERSISTENT_MAX_GROUPS; N, K > 0 and multiples of 16; row strides
 * >= K and multiples of 16, stride_bg >= (N-1)*stride_bn + K and a multiple of 16, stride_cm >= N
 * and a multiple of 8; 192*stride_am and 384*stride_bn below 2^31 - 2^16; a, b, out 16-byte
 * aligned. */
int ggemm_persistent_fp8(const void* a, const void* b, void* out, const float* a_scale, const float* b_scale,
                         const int64_t* group_offs, int32_t G, int32_t N, int32_t K, int32_t stride_am,
                         int32_t stride_bg, int32_t stride_bn, int32_t stride_cm, int32_t stride_cn,
                         int32_t a_format, int64_t M_total, void* stream);

/* Kernels behind ggemm_persistent_fp8 (same semantics; each deterministic, the two differ in
 * fp32 summation order): the 512-thread kernel of the reference's launch geometry (192-row tiles,
 * also the drop-in code objects) and a wide-tile kernel (256 threads, one wave per SIMD, 256 x 320
 * tiles, 160 KiB of LDS) for N % 320 == 0, K % 64 == 0, 256*stride_am, 320*stride_bn and
 * 512*stride_cm below 2^31 - 2^16. ggemm_persistent_fp8 runs the wide kernel wherever it applies
 * (faster at every measured shape, most on line-aligned rows of 128-byte multiples). */
#define GGEMM_PERSISTENT_KERNEL_AUTO 0
#define GGEMM_PERSISTENT_KERNEL_512 1
#define GGEMM_PERSISTENT_KERNEL_WIDE 2

/* ggemm_persistent_fp8 with the kernel chosen by the caller: GGEMM_PERSISTENT_KERNEL_AUTO (as
 * ggemm_persistent_fp8), _512 or _WIDE (GGEMM_E_SHAPE where the wide kernel does not apply). No
 * reference counterpart (the reference ships one kernel); for comparisons of the two kernels. */
int ggemm_persistent_fp8_kernel(const void* a, const void* b, void* out, const float* a_scale, const float* b_scale,
                                const int64_t* group_offs, int32_t G, int32_t N, int32_t K, int32_t stride_am,
                                int32_t stride_bg, int32_t stride_bn, int32_t stride_cm, int32_t stride_cn,
                                int32_t a_format, int64_t M_total, int32_t kernel, void* stream);

/* The kernel ggemm_persistent_fp8 runs for this shape and these strides (_512 or _WIDE). No
 * reference counterpart. */
int32_t ggemm_persistent_selected_kernel(int32_t N, int32_t K, int32_t stride_am, int32_t stride_bn,
                                         int32_t stride_cm);

/* Zeroes rows [min(offs[G], M_total), M_total) of out (bf16 [M_total, N], row stride stride_cm):
 * the rows ggemm_persistent_fp8 leaves unwritten when routing drops tokens (offs[G] < M_total).
 * offs[G] is read on the device, so the call needs no host synchronisation and can be captured in
 * a graph; with no row past offs[G] it costs one small launch. No reference counterpart (the
 * reference harness always routes every row, bench.py:205-218); the autograd layer's forward
 * output and input gradient use it so that dropped rows are exact zeros. Requirements:
 * 1 <= G <= GGEMM_PERSISTENT_MAX_GROUPS, N > 0 and a multiple of 16, 0 <= M_total < 2^31 - 256,
 * stride_cm >= N and a multiple of 8, out 16-byte aligned. */
int ggemm_persistent_clear_tail(void* out, int32_t N, int32_t stride_cm, const int64_t* group_offs, int32_t G,
                                int64_t M_total, void* stream);

/* Byte transpose of a batch of matrices: dst[b][c][r] = src[b][r][c] for b < batch, r < rows,
 * c < cols, element addresses src + b*src_bstride + r*src_rstride + c and dst + b*dst_bstride +
 * c*dst_rstride + r. For a B given [G, K, N] (N contiguous; the trans_b=False layout of the
 * Primus-Turbo API, reference bench.py:258-269) it writes the [G, N, K] operand ggemm_persistent_fp8
 * reads. No counterpart kernel in the reference, whose call sites all pass trans_b=True. rows and
 * cols multiples of 16; strides multiples of 16 with src_rstride >= cols, dst_rstride >= rows,
 * src_bstride >= rows*src_rstride, dst_bstride >= cols*dst_rstride; src and dst 16-byte aligned,
 * not overlapping. */
int ggemm_persistent_transpose_u8(const void* src, int32_t batch, int32_t rows, int32_t cols, int64_t src_bstride,
                                  int64_t src_rstride, void* dst, int64_t dst_bstride, int64_t dst_rstride,
                                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GGEMM_PERSISTENT_H */
