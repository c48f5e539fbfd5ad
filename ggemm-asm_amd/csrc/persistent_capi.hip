// extern "C" launcher of the persistent grouped FP8 GEMM (forward / data-gradient sites), part of
// libggemm_vark.so. Validates arguments on the host, then launches with the reference's geometry:
// grid (num_cus, 1, 1), block (512, 1, 1), 64 KiB dynamic LDS (reference bench.py:339-355).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/ggemm_persistent.h"
#include "capi_common.h"
#include "persistent_kernel.h"

GGEMM_DEFINE_PERSISTENT_KERNEL(_grouped_fp8_persistent_gemm_kernel, false)
GGEMM_DEFINE_PERSISTENT_KERNEL(_grouped_fp8_persistent_gemm_kernel_e5m2, true)

static_assert(GGEMM_PERSISTENT_MAX_GROUPS == ggemm::nt::kMaxGroups, "header and kernel agree");

namespace {

using ggemm::host::aligned;
using ggemm::host::device_cus;

int validate(const void* a, const void* b, const void* out, const void* as, const void* bs, const int64_t* offs,
             int G, int N, int K, int sam, int sbg, int sbn, int scm, int scn, int fmt, int64_t M_total) {
  if (!a || !b || !out || !as || !bs || !offs) return GGEMM_E_NULL;
  if (fmt != GGEMM_FP8_E4M3 && fmt != GGEMM_FP8_E5M2) return GGEMM_E_FORMAT;
  if (G <= 0 || G > ggemm::nt::kMaxGroups || N <= 0 || K <= 0 || N % 16 || K % 16) return GGEMM_E_SHAPE;
  if (M_total < 0 || M_total > ggemm::nt::kMaxRow) return GGEMM_E_SHAPE;
  // 32-bit tile indices: every group adds at most one partial M-tile
  const int64_t tiles = (M_total / ggemm::kTileM + G) * (int64_t)((N + 319) / 320);
  if (tiles > ggemm::nt::kMaxTiles) return GGEMM_E_SHAPE;
  if (scn != 1) return GGEMM_E_STRIDE;
  if (sam < K || sbn < K || sam % 16 || sbn % 16 || sbg % 16) return GGEMM_E_STRIDE;
  if ((int64_t)sbg < (int64_t)(N - 1) * sbn + K) return GGEMM_E_STRIDE;
  if (scm < N || scm % 8) return GGEMM_E_STRIDE;
  // 32-bit buffer offsets of a stage: 192 A rows, up to 384 B rows, below the out-of-range offset
  if ((int64_t)sam * ggemm::kTileM >= ggemm::nt::kOob || (int64_t)sbn * 384 >= ggemm::nt::kOob)
    return GGEMM_E_SHAPE;
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(out, 16)) return GGEMM_E_ALIGN;
  return GGEMM_OK;
}

}  // namespace

extern "C" {

int ggemm_persistent_fp8(const void* a, const void* b, void* out, const float* a_scale, const float* b_scale,
                         const int64_t* group_offs, int32_t G, int32_t N, int32_t K, int32_t stride_am,
                         int32_t stride_bg, int32_t stride_bn, int32_t stride_cm, int32_t stride_cn,
                         int32_t a_format, int64_t M_total, void* stream) {
  int rc = validate(a, b, out, a_scale, b_scale, group_offs, G, N, K, stride_am, stride_bg, stride_bn, stride_cm,
                    stride_cn, a_format, M_total);
  if (rc) return rc;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  if (M_total == 0) return GGEMM_OK;   // no rows: nothing to write
  auto kern = a_format == GGEMM_FP8_E5M2 ? _grouped_fp8_persistent_gemm_kernel_e5m2
                                         : _grouped_fp8_persistent_gemm_kernel;
  hipLaunchKernelGGL(kern, dim3(cus), dim3(ggemm::kThreads), ggemm::kDynLdsBytes, (hipStream_t)stream,
                     (const uint8_t*)a, (const uint8_t*)b, (uint16_t*)out, a_scale, b_scale, group_offs, G, N, K,
                     stride_am, stride_bg, stride_bn, stride_cm, stride_cn, (void*)nullptr, (void*)nullptr);
  return (int)hipGetLastError();
}

}  // extern "C"
