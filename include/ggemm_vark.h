/* C ABI of the MI355X variable-K FP8 grouped weight-gradient library (libggemm_vark.so).
 *
 *   C[g] = s_lhs * s_rhs * LHS[offs[g]:offs[g+1], :]^T @ RHS[offs[g]:offs[g+1], :]
 *
 * All pointers are device pointers except where stated; sizes and strides are in elements.
 * Every entry point returns 0 on success, a positive hipError_t value when the HIP runtime
 * failed, or a negative GGEMM_E_* code when argument validation failed (nothing is launched
 * then). Launches are asynchronous on `stream` (a hipStream_t; NULL = the null stream).
 * No entry point allocates device memory, keeps state between calls, or synchronizes.
 */
#ifndef GGEMM_VARK_H
#define GGEMM_VARK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGEMM_VARK_ABI_VERSION 9

enum {
  GGEMM_OK = 0,
  GGEMM_E_NULL = -1,        /* a required pointer is NULL */
  GGEMM_E_SHAPE = -2,       /* G, OUT_M or OUT_N <= 0, OUT_M/OUT_N not multiples of 16, row strides
                               too large for 32-bit stage offsets, or more than 2^30 output tiles */
  GGEMM_E_STRIDE = -3,      /* strides too small, stride_cn != 1, or not multiples of 16 / 4 */
  GGEMM_E_ALIGN = -4,       /* LHS/RHS not 16-byte aligned or C not 8-byte aligned */
  GGEMM_E_OFFSETS = -5,     /* host group offsets not 0-based, non-decreasing, or past M_total */
  GGEMM_E_DEVICE = -6,      /* no usable device / not a gfx950 device */
  GGEMM_E_MX_ALIGN = -7,    /* MX: a group does not start on a 32-token block boundary */
  GGEMM_E_FORMAT = -8       /* unknown fp8 format code (ggemm_persistent.h) */
};

/* Tensorwise FP8 grouped wgrad. Replaces the reference's code-object launch of
 * `_grouped_variable_k_gemm_kernel` (reference bench.py:364-413 prepare_variable_k_args /
 * launch_variable_k_kernel, launcher.cpp:123-171) and the Triton op it stands in for
 * (reference bench.py:268, `_triton_vark(lhs, rhs, lhs_scale, rhs_scale, group_offs)`).
 * lhs: e4m3fn [M_total, OUT_M] (row stride stride_lhs_m); rhs: e5m2 [M_total, OUT_N]
 * (row stride stride_rhs_m); out: bf16 [G, OUT_M, OUT_N] (strides stride_cg, stride_cm,
 * stride_cn == 1); lhs_scale / rhs_scale: fp32 scalars; group_offs: int64 [G+1], offs[0] = 0,
 * non-decreasing, offs[G] <= M_total (the caller's guarantee, as with the reference kernel: this
 * argument list carries no token count; ggemm_vark_wgrad_fp8_out with GGEMM_OUT_BF16 is the same
 * launch bounded by M_total). Every element of out[0:G] is written, empty groups with zeros.
 * Requirements: OUT_M, OUT_N, stride_lhs_m, stride_rhs_m multiples of 16; stride_cm,
 * stride_cg multiples of 4; lhs/rhs 16-byte aligned, out 8-byte aligned. A token row of lhs / rhs
 * may be read up to its stride, padding included, so with a padded row stride the last row must
 * be allocated in full (M_total * stride bytes from the base), as a view into a wider tensor is.
 * The same holds for every wgrad entry below. */
int ggemm_vark_wgrad_fp8(const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                         const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                         int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                         int32_t stride_cm, int32_t stride_cn, void* stream);

/* Same as ggemm_vark_wgrad_fp8 but with the K=32 MFMA (v_mfma_f32_16x16x32_bf8_fp8) the
 * reference kernel is built on (reference README.md:5). Kept to measure the instruction choice;
 * same contract and results within fp32 accumulation order. */
int ggemm_vark_wgrad_fp8_k32(const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                             const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                             int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                             int32_t stride_cm, int32_t stride_cn, void* stream);

/* Output modes of ggemm_vark_wgrad_fp8_out. */
#define GGEMM_OUT_BF16 0        /* C bf16 (ggemm_vark_wgrad_fp8) */
#define GGEMM_OUT_F32 1         /* C fp32: C[g] = s_lhs s_rhs LHS_g^T RHS_g, no bf16 rounding */
#define GGEMM_OUT_F32_ACCUM 2   /* C fp32, accumulated in place: C[g] += s_lhs s_rhs LHS_g^T RHS_g */

/* Tensorwise FP8 grouped wgrad with a chosen output: the fp32 modes write (or, with
 * GGEMM_OUT_F32_ACCUM, add into) an fp32 C [G, OUT_M, OUT_N] -- the main-grad accumulation of a
 * training step (beta = 1), with the product rounded once to fp32 before the addition. No
 * reference counterpart: the reference kernel writes bf16 only (reference launcher.cpp:16-33);
 * the modes are the epilogue variants a training framework needs around it. Same arguments as
 * ggemm_vark_wgrad_fp8 with strides in elements of C's type, plus M_total >= 0, the token count
 * of lhs and rhs: every group offset is clamped to [0, M_total] on the device, so no load leaves
 * the tensors whatever group_offs holds (group g covers tokens [clamp(offs[g]), clamp(offs[g+1]))).
 * fp32 C must be 16-byte aligned, stride_cm and stride_cg multiples of 4. Accumulate mode reads
 * and writes every element of C[0:G] once per launch (empty groups add zero), so a launch is
 * deterministic. GGEMM_OUT_BF16 is ggemm_vark_wgrad_fp8 bounded by M_total. */
int ggemm_vark_wgrad_fp8_out(const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                             const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                             int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                             int32_t stride_cm, int32_t stride_cn, int32_t out_mode, int64_t M_total,
                             void* stream);

/* Tensorwise FP8 grouped wgrad on a wide-tile kernel: 320 x 320 or 256 x 384 output tiles on
 * 256-thread workgroups (one wave per SIMD, 512 registers per wave), outside the reference's
 * 512-thread launch contract; no reference counterpart (it replaces the same launch as
 * ggemm_vark_wgrad_fp8, reference launcher.cpp:123-171, for the shapes it takes). Same arguments
 * and result as ggemm_vark_wgrad_fp8_out with the same out_mode, group offsets clamped to
 * [0, min(M_total, 2^31 - 1)]. tile_m: 320 (OUT_M and OUT_N multiples of 320), 256 (OUT_N a
 * multiple of 384; bf16 C only) or 0 (320 where it fits, else 256). Also a group of C within 2^31
 * bytes, and every C row and group starting on 16 bytes (out 16-byte aligned, stride_cm and
 * stride_cg multiples of 8 for bf16 C, of 4 for fp32 C: the epilogue stores 16-byte row chunks);
 * otherwise GGEMM_E_SHAPE / GGEMM_E_ALIGN / GGEMM_E_FORMAT and nothing is launched. */
int ggemm_vark_wgrad_fp8_wide(const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                              const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                              int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                              int32_t stride_cm, int32_t stride_cn, int64_t M_total, int32_t tile_m,
                              int32_t out_mode, void* stream);

/* MXFP8 block-scaled grouped wgrad (no reference counterpart: the reference imports only the
 * tensorwise kernels, reference bench.py:241-246). lhs_scale: e8m0 bytes [ceil(M_total/32), OUT_M]
 * with row stride stride_lhs_scale; rhs_scale: e8m0 [ceil(M_total/32), OUT_N], row stride
 * stride_rhs_scale. Token block b (tokens 32b..32b+31) of a column is multiplied by
 * 2^(scale[b][col]-127). Every group must start at a multiple of 32 tokens (ggemm_vark_check_offsets
 * with mx = 1 checks a host copy; otherwise the caller's responsibility). Group offsets are
 * clamped to [0, M_total] on the device, as in ggemm_vark_wgrad_fp8_out. Runs the 320 x 320
 * wide-tile kernel where ggemm_vark_bf16_kernel returns 320 for the shape, else the 192-row one. */
int ggemm_vark_wgrad_mxfp8(const void* lhs, const void* rhs, void* out, const uint8_t* lhs_scale,
                           const uint8_t* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                           int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                           int32_t stride_cm, int32_t stride_cn, int32_t stride_lhs_scale,
                           int32_t stride_rhs_scale, int64_t M_total, void* stream);

/* ggemm_vark_wgrad_mxfp8 on a chosen kernel (no reference counterpart): tile_m 320 = the 320 x 320
 * wide-tile kernel (OUT_M and OUT_N multiples of 320, a group of C within 2^31 bytes, out 16-byte
 * aligned, stride_cm and stride_cg multiples of 8, group offsets clamped to
 * [0, min(M_total, 2^31 - 1)]; otherwise GGEMM_E_SHAPE /
 * GGEMM_E_ALIGN and nothing is launched), 192 = the 192-row-tile kernel, 0 = the choice of
 * ggemm_vark_wgrad_mxfp8. Same arguments and result otherwise. */
int ggemm_vark_wgrad_mxfp8_tile(const void* lhs, const void* rhs, void* out, const uint8_t* lhs_scale,
                                const uint8_t* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                                int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                                int32_t stride_cm, int32_t stride_cn, int32_t stride_lhs_scale,
                                int32_t stride_rhs_scale, int64_t M_total, int32_t tile_m, void* stream);

/* Host-side check of a group-offset array (host memory, G+1 entries) against M_total; MX also
 * checks 32-token alignment of group starts. Mirrors the invariants the reference generator
 * asserts (reference bench.py:211,215-218). Returns GGEMM_OK, GGEMM_E_OFFSETS or
 * GGEMM_E_MX_ALIGN. Touches no device. */
int ggemm_vark_check_offsets(const int64_t* host_group_offs, int32_t G, int64_t M_total, int32_t mx);

/* Number of compute units of `device` (the persistent grid size; reference launcher.cpp:78-81,
 * bench.py:226-228). */
int ggemm_vark_num_cus(int32_t device, int32_t* num_cus);

/* Static human-readable text for a return code of this library (HIP codes included). */
const char* ggemm_vark_strerror(int32_t code);

/* GGEMM_VARK_ABI_VERSION of the loaded library. */
int32_t ggemm_vark_abi_version(void);

/* Which kernel the bf16 entry points (ggemm_vark_wgrad_fp8, ggemm_vark_wgrad_fp8_out with
 * GGEMM_OUT_BF16) run for a shape: 320 or 256 = the wide-tile kernel with that tile height
 * (OUT_M >= 1024, a shape ggemm_vark_wgrad_fp8_wide takes with tile_m = 0, out 16-byte aligned,
 * stride_cm a multiple of 8; groups contiguous, stride_cg = OUT_M * stride_cm, which the entry
 * points also require to be a multiple of 8 for a wide kernel), 0 = the 192-row-tile kernel of the
 * reference launch geometry. The fp32 modes of ggemm_vark_wgrad_fp8_out run the 320 x 320 kernel
 * where this returns 320 for stride_cm twice the fp32 row stride, ggemm_vark_wgrad_mxfp8 its MX
 * variant where this returns 320. No reference counterpart. Touches no device. */
int32_t ggemm_vark_bf16_kernel(int32_t OUT_M, int32_t OUT_N, int32_t stride_cm, const void* out);

/* Launch geometry the library uses (and the drop-in code object expects) for a problem of width
 * OUT_N = out_n: block threads, dynamic LDS bytes, output tile (OUT_M x OUT_N; the N tile is 384
 * when out_n is a multiple of 384, else 320) and tokens per pipeline stage. */
void ggemm_vark_launch_geometry(int32_t out_n, int32_t* block_threads, int32_t* dynamic_lds, int32_t* tile_m,
                                int32_t* tile_n, int32_t* k_step);

#ifdef __cplusplus
}
#endif

#endif /* GGEMM_VARK_H */
