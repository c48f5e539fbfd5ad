// extern "C" launcher library for the variable-K FP8 grouped wgrad kernels (libggemm_vark.so).
// Validates arguments on the host, then launches the persistent kernel with the reference's
// geometry: grid (num_cus, 1, 1), block (512, 1, 1), 64 KiB dynamic LDS
// (reference launcher.cpp:142-171, bench.py:388-398).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/ggemm_vark.h"
#include "capi_common.h"
#include "vark_kernel.h"
#include "vark_wide.h"

GGEMM_DEFINE_TENSORWISE_LIB_KERNEL(_grouped_variable_k_gemm_kernel, false, uint16_t, ggemm::kOutBF16)
GGEMM_DEFINE_TENSORWISE_LIB_KERNEL(_grouped_variable_k_gemm_kernel_k32, true, uint16_t, ggemm::kOutBF16)
GGEMM_DEFINE_MX_KERNEL(_grouped_variable_k_mxfp8_gemm_kernel)
GGEMM_DEFINE_TENSORWISE_LIB_KERNEL(_grouped_variable_k_gemm_kernel_f32, false, float, ggemm::kOutF32)
GGEMM_DEFINE_TENSORWISE_LIB_KERNEL(_grouped_variable_k_gemm_kernel_f32_acc, false, float, ggemm::kOutF32Acc)
GGEMM_DEFINE_WIDE_KERNEL(_grouped_variable_k_gemm_kernel_wide, 256, 384, uint16_t, ggemm::kOutBF16)
GGEMM_DEFINE_WIDE_KERNEL(_grouped_variable_k_gemm_kernel_wide320, 320, 320, uint16_t, ggemm::kOutBF16)
GGEMM_DEFINE_WIDE_KERNEL(_grouped_variable_k_gemm_kernel_wide320_f32, 320, 320, float, ggemm::kOutF32)
GGEMM_DEFINE_WIDE_KERNEL(_grouped_variable_k_gemm_kernel_wide320_f32_acc, 320, 320, float, ggemm::kOutF32Acc)
GGEMM_DEFINE_WIDE_MX_KERNEL(_grouped_variable_k_mxfp8_gemm_kernel_wide320)

namespace {

using ggemm::host::aligned;
using ggemm::host::device_cus;

int validate_common(const void* lhs, const void* rhs, const void* out, const void* ls, const void* rs,
                    const int64_t* offs, int G, int OUT_M, int OUT_N, int slm, int srm, int scg, int scm,
                    int scn) {
  if (!lhs || !rhs || !out || !ls || !rs || !offs) return GGEMM_E_NULL;
  if (G <= 0 || OUT_M <= 0 || OUT_N <= 0) return GGEMM_E_SHAPE;
  if (OUT_M % 16 || OUT_N % 16) return GGEMM_E_SHAPE;
  if (scn != 1) return GGEMM_E_STRIDE;
  if (slm < OUT_M || srm < OUT_N || slm % 16 || srm % 16) return GGEMM_E_STRIDE;
  if (scm < OUT_N || scm % 4 || scg % 4) return GGEMM_E_STRIDE;
  if ((int64_t)scg < (int64_t)(OUT_M - 1) * scm + OUT_N) return GGEMM_E_STRIDE;
  // the kernel forms 32-bit buffer offsets of up to 128 rows of a stage
  if ((int64_t)slm * 129 > INT32_MAX || (int64_t)srm * 129 > INT32_MAX) return GGEMM_E_SHAPE;
  // ... and 32-bit tile indices: at most 2^30 output tiles (counted with the narrower 320 tile)
  const int64_t tiles = (int64_t)((OUT_M + ggemm::kTileM - 1) / ggemm::kTileM) * ((OUT_N + 319) / 320);
  if ((int64_t)G * tiles > (int64_t(1) << 30)) return GGEMM_E_SHAPE;
  if (!aligned(lhs, 16) || !aligned(rhs, 16) || !aligned(out, 8)) return GGEMM_E_ALIGN;
  return GGEMM_OK;
}

// Wide-tile kernels (tile = its OUT_M height): 320 x 320 where it divides both output dims (no
// partial tiles), else 256 x 384 where OUT_N is a multiple of 384 (N-ragged tiles would need
// per-lane store masks; rows past OUT_M fall outside the C buffer resource); a group of C must be
// addressable with 32-bit byte offsets. 0: no wide kernel takes the shape.
int wide_tile_for(int OUT_M, int OUT_N, int scm) {
  if ((int64_t)OUT_M * scm * 2 >= INT32_MAX) return 0;
  if (OUT_M % 320 == 0 && OUT_N % 320 == 0) return 320;
  if (OUT_N % 384 == 0) return 256;
  return 0;
}

// The wide kernels' epilogues store 16-byte chunks of C rows: every row and group must start on 16
// bytes. scm / scg in bf16 elements (twice the fp32 strides for an fp32 C).
bool wide_rows_aligned(const void* out, int64_t scm, int64_t scg) {
  return aligned(out, 16) && scm % 8 == 0 && scg % 8 == 0;
}

// The bf16 entry points run a wide-tile kernel where one takes the shape, C rows start on 16 bytes
// and the problem is large enough to fill its tiles (OUT_M >= 1024); otherwise the 192 x 384 /
// 192 x 320 kernel.
int wide_selected(int OUT_M, int OUT_N, int64_t scm, int64_t scg, const void* out) {
  return OUT_M >= 1024 && wide_rows_aligned(out, scm, scg) ? wide_tile_for(OUT_M, OUT_N, (int)scm) : 0;
}

int launch_wide(int tile, int out_mode, const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M, int32_t OUT_N,
                int32_t slm, int32_t srm, int32_t scg, int32_t scm, int32_t scn, int64_t M_total, void* stream) {
  int cus = 0;
  int rc = device_cus(&cus);
  if (rc) return rc;
  // the kernels keep token counts in 32 bits: a group never exceeds 2^31 - 1 tokens
  const int64_t m_total = M_total < INT32_MAX ? M_total : INT32_MAX;
  const dim3 grid(cus), block(ggemm::wide::kNT);
  if (out_mode == GGEMM_OUT_BF16) {
    auto kern = tile == 320 ? _grouped_variable_k_gemm_kernel_wide320 : _grouped_variable_k_gemm_kernel_wide;
    hipLaunchKernelGGL(kern, grid, block, 0, (hipStream_t)stream, (const uint8_t*)lhs, (const uint8_t*)rhs,
                       (uint16_t*)out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, slm, srm, scg, scm, scn,
                       (void*)nullptr, (void*)nullptr, m_total);
  } else {
    auto kern = out_mode == GGEMM_OUT_F32 ? _grouped_variable_k_gemm_kernel_wide320_f32
                                          : _grouped_variable_k_gemm_kernel_wide320_f32_acc;
    hipLaunchKernelGGL(kern, grid, block, 0, (hipStream_t)stream, (const uint8_t*)lhs, (const uint8_t*)rhs,
                       (float*)out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, slm, srm, scg, scm, scn,
                       (void*)nullptr, (void*)nullptr, m_total);
  }
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

// m_total: the token count group offsets are clamped to on the device (INT64_MAX for the entry
// points with the reference's argument list, which carries none).
static int launch_tensorwise(bool legacy, const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                             const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                             int32_t OUT_N, int32_t slm, int32_t srm, int32_t scg, int32_t scm, int32_t scn,
                             int64_t m_total, void* stream) {
  int rc = validate_common(lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, slm, srm, scg, scm,
                           scn);
  if (rc) return rc;
  if (m_total < 0) return GGEMM_E_SHAPE;
  if (const int tile = legacy ? 0 : wide_selected(OUT_M, OUT_N, scm, scg, out))
    return launch_wide(tile, GGEMM_OUT_BF16, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, slm,
                       srm, scg, scm, scn, m_total, stream);
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  auto kern = legacy ? _grouped_variable_k_gemm_kernel_k32 : _grouped_variable_k_gemm_kernel;
  hipLaunchKernelGGL(kern, dim3(cus), dim3(ggemm::kThreads), ggemm::kDynLdsBytes, (hipStream_t)stream,
                     (const uint8_t*)lhs, (const uint8_t*)rhs, (uint16_t*)out, lhs_scale, rhs_scale, group_offs, G,
                     OUT_M, OUT_N, slm, srm, scg, scm, scn, (void*)nullptr, (void*)nullptr, m_total);
  return (int)hipGetLastError();
}

int ggemm_vark_wgrad_fp8_wide(const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                              const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                              int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                              int32_t stride_cm, int32_t stride_cn, int64_t M_total, int32_t tile_m,
                              int32_t out_mode, void* stream) {
  if (out_mode != GGEMM_OUT_BF16 && out_mode != GGEMM_OUT_F32 && out_mode != GGEMM_OUT_F32_ACCUM)
    return GGEMM_E_FORMAT;
  int rc = validate_common(lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                           stride_rhs_m, stride_cg, stride_cm, stride_cn);
  if (rc) return rc;
  if (M_total < 0) return GGEMM_E_SHAPE;
  // fp32 C: the same byte bound as a bf16 C twice as wide
  const int fit = wide_tile_for(OUT_M, OUT_N, out_mode == GGEMM_OUT_BF16 ? stride_cm : 2 * stride_cm);
  int tile = tile_m == 0 ? fit : tile_m;
  if (tile == 320 && (OUT_M % 320 || OUT_N % 320)) tile = 0;
  if (tile == 256 && (OUT_N % 384 || out_mode != GGEMM_OUT_BF16)) tile = 0;   // fp32 epilogues: 320 x 320
  if ((tile != 256 && tile != 320) || fit == 0) return GGEMM_E_SHAPE;
  const int64_t w = out_mode == GGEMM_OUT_BF16 ? 1 : 2;   // strides in bf16 elements
  if (!wide_rows_aligned(out, w * stride_cm, w * stride_cg)) return GGEMM_E_ALIGN;   // 16-byte row chunks
  return launch_wide(tile, out_mode, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                     stride_rhs_m, stride_cg, stride_cm, stride_cn, M_total, stream);
}

int ggemm_vark_wgrad_fp8(const void* lhs, const void* rhs, void* out, const float* lhs_scale, const float* rhs_scale,
                         const int64_t* group_offs, int32_t G, int32_t OUT_M, int32_t OUT_N, int32_t stride_lhs_m,
                         int32_t stride_rhs_m, int32_t stride_cg, int32_t stride_cm, int32_t stride_cn,
                         void* stream) {
  return launch_tensorwise(false, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                           stride_rhs_m, stride_cg, stride_cm, stride_cn, INT64_MAX, stream);
}

int ggemm_vark_wgrad_fp8_k32(const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                             const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                             int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                             int32_t stride_cm, int32_t stride_cn, void* stream) {
  return launch_tensorwise(true, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                           stride_rhs_m, stride_cg, stride_cm, stride_cn, INT64_MAX, stream);
}

int ggemm_vark_wgrad_fp8_out(const void* lhs, const void* rhs, void* out, const float* lhs_scale,
                             const float* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                             int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                             int32_t stride_cm, int32_t stride_cn, int32_t out_mode, int64_t M_total,
                             void* stream) {
  if (out_mode == GGEMM_OUT_BF16)
    return launch_tensorwise(false, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                             stride_rhs_m, stride_cg, stride_cm, stride_cn, M_total, stream);
  if (out_mode != GGEMM_OUT_F32 && out_mode != GGEMM_OUT_F32_ACCUM) return GGEMM_E_FORMAT;
  int rc = validate_common(lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                           stride_rhs_m, stride_cg, stride_cm, stride_cn);
  if (rc) return rc;
  if (M_total < 0) return GGEMM_E_SHAPE;
  if (!aligned(out, 16)) return GGEMM_E_ALIGN;    // 16-byte fp32 row segments
  // fp32 C takes the 320 x 320 wide-tile kernel where the bf16 C of the same shape would
  if (wide_selected(OUT_M, OUT_N, 2 * (int64_t)stride_cm, 2 * (int64_t)stride_cg, out) == 320)
    return launch_wide(320, out_mode, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N,
                       stride_lhs_m, stride_rhs_m, stride_cg, stride_cm, stride_cn, M_total, stream);
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  auto kern = out_mode == GGEMM_OUT_F32 ? _grouped_variable_k_gemm_kernel_f32 : _grouped_variable_k_gemm_kernel_f32_acc;
  hipLaunchKernelGGL(kern, dim3(cus), dim3(ggemm::kThreads), ggemm::kDynLdsBytes, (hipStream_t)stream,
                     (const uint8_t*)lhs, (const uint8_t*)rhs, (float*)out, lhs_scale, rhs_scale, group_offs, G, OUT_M,
                     OUT_N, stride_lhs_m, stride_rhs_m, stride_cg, stride_cm, stride_cn, (void*)nullptr, (void*)nullptr,
                     M_total);
  return (int)hipGetLastError();
}

// tile_m: 0 = the wide 320 x 320 kernel where the bf16 tensorwise entry would run it, else the
// 192-row kernel; 320 / 192 = that kernel (320 only for shapes it takes)
static int launch_mx(int32_t tile_m, const void* lhs, const void* rhs, void* out, const uint8_t* lhs_scale,
                     const uint8_t* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M, int32_t OUT_N,
                     int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg, int32_t stride_cm,
                     int32_t stride_cn, int32_t stride_lhs_scale, int32_t stride_rhs_scale, int64_t M_total,
                     void* stream) {
  int rc = validate_common(lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                           stride_rhs_m, stride_cg, stride_cm, stride_cn);
  if (rc) return rc;
  if (M_total < 0) return GGEMM_E_SHAPE;
  if (stride_lhs_scale < OUT_M || stride_rhs_scale < OUT_N || stride_lhs_scale % 16 || stride_rhs_scale % 16)
    return GGEMM_E_STRIDE;
  if (!aligned(lhs_scale, 16) || !aligned(rhs_scale, 16)) return GGEMM_E_ALIGN;
  if (tile_m != 0 && tile_m != 320 && tile_m != 192) return GGEMM_E_SHAPE;
  bool wide = tile_m == 0 ? wide_selected(OUT_M, OUT_N, stride_cm, stride_cg, out) == 320 : tile_m == 320;
  if (tile_m == 320) {
    if (wide_tile_for(OUT_M, OUT_N, stride_cm) != 320) return GGEMM_E_SHAPE;
    if (!wide_rows_aligned(out, stride_cm, stride_cg)) return GGEMM_E_ALIGN;    // 16-byte row chunks
  }
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  if (wide) {
    // the kernels keep token counts in 32 bits: a group never exceeds 2^31 - 1 tokens
    const int64_t m_total = M_total < INT32_MAX ? M_total : INT32_MAX;
    hipLaunchKernelGGL(_grouped_variable_k_mxfp8_gemm_kernel_wide320, dim3(cus), dim3(ggemm::wide::kNT), 0,
                       (hipStream_t)stream, (const uint8_t*)lhs, (const uint8_t*)rhs, (uint16_t*)out, lhs_scale,
                       rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m, stride_rhs_m, stride_cg, stride_cm,
                       stride_cn, stride_lhs_scale, stride_rhs_scale, m_total);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(_grouped_variable_k_mxfp8_gemm_kernel, dim3(cus), dim3(ggemm::kThreads), ggemm::kDynLdsBytes,
                     (hipStream_t)stream, (const uint8_t*)lhs, (const uint8_t*)rhs, (uint16_t*)out, lhs_scale,
                     rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m, stride_rhs_m, stride_cg, stride_cm,
                     stride_cn, stride_lhs_scale, stride_rhs_scale, (void*)nullptr, (void*)nullptr, M_total);
  return (int)hipGetLastError();
}

int ggemm_vark_wgrad_mxfp8(const void* lhs, const void* rhs, void* out, const uint8_t* lhs_scale,
                           const uint8_t* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                           int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                           int32_t stride_cm, int32_t stride_cn, int32_t stride_lhs_scale, int32_t stride_rhs_scale,
                           int64_t M_total, void* stream) {
  return launch_mx(0, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m, stride_rhs_m,
                   stride_cg, stride_cm, stride_cn, stride_lhs_scale, stride_rhs_scale, M_total, stream);
}

int ggemm_vark_wgrad_mxfp8_tile(const void* lhs, const void* rhs, void* out, const uint8_t* lhs_scale,
                                const uint8_t* rhs_scale, const int64_t* group_offs, int32_t G, int32_t OUT_M,
                                int32_t OUT_N, int32_t stride_lhs_m, int32_t stride_rhs_m, int32_t stride_cg,
                                int32_t stride_cm, int32_t stride_cn, int32_t stride_lhs_scale,
                                int32_t stride_rhs_scale, int64_t M_total, int32_t tile_m, void* stream) {
  return launch_mx(tile_m, lhs, rhs, out, lhs_scale, rhs_scale, group_offs, G, OUT_M, OUT_N, stride_lhs_m,
                   stride_rhs_m, stride_cg, stride_cm, stride_cn, stride_lhs_scale, stride_rhs_scale, M_total, stream);
}

int ggemm_vark_check_offsets(const int64_t* offs, int32_t G, int64_t M_total, int32_t mx) {
  if (!offs || G <= 0) return GGEMM_E_OFFSETS;
  if (offs[0] != 0) return GGEMM_E_OFFSETS;
  for (int g = 0; g < G; ++g) {
    if (offs[g + 1] < offs[g]) return GGEMM_E_OFFSETS;
    if (mx && (offs[g] % 32)) return GGEMM_E_MX_ALIGN;
  }
  if (offs[G] > M_total) return GGEMM_E_OFFSETS;
  return GGEMM_OK;
}

int ggemm_vark_num_cus(int32_t device, int32_t* num_cus) {
  if (!num_cus) return GGEMM_E_NULL;
  int v = 0;
  hipError_t e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return (int)e;
  *num_cus = v;
  return GGEMM_OK;
}

const char* ggemm_vark_strerror(int32_t code) {
  switch (code) {
    case GGEMM_OK: return "success";
    case GGEMM_E_NULL: return "a required pointer is NULL";
    case GGEMM_E_SHAPE:
      return "invalid shape (G, OUT_M, OUT_N must be > 0, OUT_M/OUT_N multiples of 16, row strides below "
             "2^31/129, at most 2^30 output tiles)";
    case GGEMM_E_STRIDE: return "invalid strides (row strides >= width and multiples of 16, stride_cn == 1)";
    case GGEMM_E_ALIGN: return "misaligned pointer (LHS/RHS 16-byte, C 8-byte)";
    case GGEMM_E_OFFSETS: return "invalid group offsets (must start at 0, be non-decreasing, end <= M_total)";
    case GGEMM_E_DEVICE: return "current device is not a usable gfx950 (MI355X) GPU";
    case GGEMM_E_MX_ALIGN: return "MXFP8 groups must start on 32-token block boundaries";
    case GGEMM_E_FORMAT: return "unknown fp8 format code (A: GGEMM_FP8_E4M3 or GGEMM_FP8_E5M2)";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown error";
}

int32_t ggemm_vark_abi_version(void) { return GGEMM_VARK_ABI_VERSION; }

int32_t ggemm_vark_bf16_kernel(int32_t OUT_M, int32_t OUT_N, int32_t stride_cm, const void* out) {
  return wide_selected(OUT_M, OUT_N, stride_cm, (int64_t)OUT_M * stride_cm, out);
}

void ggemm_vark_launch_geometry(int32_t out_n, int32_t* block_threads, int32_t* dynamic_lds, int32_t* tile_m,
                                int32_t* tile_n, int32_t* k_step) {
  if (block_threads) *block_threads = ggemm::kThreads;
  if (dynamic_lds) *dynamic_lds = ggemm::kDynLdsBytes;
  if (tile_m) *tile_m = ggemm::kTileM;
  if (tile_n) *tile_n = (out_n > 0 && ggemm::wide_tiles(out_n, false)) ? 384 : 320;
  if (k_step) *k_step = ggemm::kKStep;
}

}  // extern "C"
