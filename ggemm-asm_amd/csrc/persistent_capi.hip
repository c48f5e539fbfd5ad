// extern "C" launcher of the persistent grouped FP8 GEMM (forward / data-gradient sites), part of
// libggemm_vark.so. Validates arguments on the host, then launches either the kernel of the
// reference's geometry (grid (num_cus, 1, 1), block (512, 1, 1), 64 KiB dynamic LDS, reference
// bench.py:339-355) or, for the shapes it takes, the wide-tile kernel (persistent_wide.h: grid
// (num_cus, 1, 1), block (256, 1, 1), 160 KiB static LDS).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/ggemm_persistent.h"
#include "capi_common.h"
#include "persistent_kernel.h"
#include "persistent_wide.h"
#include "transpose_tile.h"

GGEMM_DEFINE_PERSISTENT_LIB_KERNEL(_grouped_fp8_persistent_gemm_kernel, false)
GGEMM_DEFINE_PERSISTENT_LIB_KERNEL(_grouped_fp8_persistent_gemm_kernel_e5m2, true)
GGEMM_DEFINE_PERSISTENT_WIDE_KERNEL(_grouped_fp8_persistent_gemm_kernel_wide, false)
GGEMM_DEFINE_PERSISTENT_WIDE_KERNEL(_grouped_fp8_persistent_gemm_kernel_wide_e5m2, true)

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

// Byte transpose over 128 x 128 tiles (ggemm_persistent_transpose_u8), the tile scheme of the
// quantize-and-transpose producer (transpose_tile.h: LDS map tt_off, byte_col): thread t loads 16
// bytes of each of the tile rows t / 8 + 32h (h = 0..3, all loads issued first) into the LDS tile;
// after a barrier it reads the dwords of tile columns 4 (t / 8) .. +3 in tile rows 16 (t % 8) ..
// +15 and writes 16 bytes to each of those four destination rows, so a store instruction's 8
// threads of a column group write one whole 128-byte line. Edge tiles hold whole 16-byte segments.
constexpr int kXT = 128, kXThreads = 256;
typedef unsigned int xv4u __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(kXThreads) transpose_u8_kernel(const uint8_t* src, int batch, int rows, int cols,
                                                                 int64_t sb, int64_t sr, uint8_t* dst, int64_t db,
                                                                 int64_t dr) {
  __shared__ __attribute__((aligned(16))) uint8_t s_t[kXT * kXT];
  const int tid = threadIdx.x;
  const int tr = tid >> 3, tc = 16 * (tid & 7);
  const int cg = tid >> 3, rj = tid & 7;
  const int rt = (rows + kXT - 1) / kXT, ct = (cols + kXT - 1) / kXT;
  const int per = rt * ct;
  const int64_t tiles = (int64_t)batch * per;
  for (int64_t it = blockIdx.x; it < tiles; it += gridDim.x) {
    const int b = (int)(it / per);
    const int rem = (int)(it - (int64_t)b * per);
    const int r0 = (rem / ct) * kXT, c0 = (rem % ct) * kXT;
    xv4u v[4];
#pragma unroll
    for (int h = 0; h < 4; ++h)
      if (c0 + tc < cols && r0 + tr + 32 * h < rows)
        v[h] = __builtin_nontemporal_load((const xv4u*)(src + b * sb + (int64_t)(r0 + tr + 32 * h) * sr + c0 + tc));
#pragma unroll
    for (int h = 0; h < 4; ++h)
      if (c0 + tc < cols && r0 + tr + 32 * h < rows) *(xv4u*)(s_t + ggemm::qt::tt_off(tr + 32 * h, tc)) = v[h];
    __syncthreads();
    if (r0 + 16 * rj < rows && c0 + 4 * cg < cols) {
      uint32_t dw[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) dw[i] = *(const uint32_t*)(s_t + ggemm::qt::tt_off(16 * rj + i, 4 * cg));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        using ggemm::qt::byte_col;
        uint8_t* out = dst + b * db + (int64_t)(c0 + 4 * cg + k) * dr + r0 + 16 * rj;
        __builtin_nontemporal_store(xv4u{byte_col(dw[0], dw[1], dw[2], dw[3], k), byte_col(dw[4], dw[5], dw[6], dw[7], k),
                                          byte_col(dw[8], dw[9], dw[10], dw[11], k),
                                          byte_col(dw[12], dw[13], dw[14], dw[15], k)},
                                    (xv4u*)out);
      }
    }
    __syncthreads();
  }
}

// Zeroes rows [clamp(offs[G]), m_total) of a bf16 [m_total, N] output (ggemm_persistent_clear_tail):
// the row range comes from the device copy of the offsets, so no host synchronisation is needed;
// rows are dealt to workgroups round robin, 16-byte chunks of a row to threads (N is a multiple of
// 16, rows 16-byte aligned).
constexpr int kTailThreads = 256;

__global__ void __launch_bounds__(kTailThreads) clear_tail_kernel(uint16_t* out, int64_t stride_cm, int N,
                                                                  const int64_t* group_offs, int G,
                                                                  int64_t m_total) {
  int64_t r0 = group_offs[G];
  r0 = r0 < 0 ? 0 : (r0 > m_total ? m_total : r0);
  const int chunks = N / 8;
  for (int64_t r = r0 + blockIdx.x; r < m_total; r += gridDim.x) {
    xv4u* row = reinterpret_cast<xv4u*>(out + r * stride_cm);
    for (int c = threadIdx.x; c < chunks; c += kTailThreads) row[c] = xv4u{0u, 0u, 0u, 0u};
  }
}

// The wide-tile kernel takes N % 320 == 0 and K % 64 == 0 (persistent_wide.h); its 32-bit buffer
// offsets: 256 A rows and 320 B rows per stage below the out-of-range offset, a C tile's 256 rows
// within num_records.
bool wide_fits(int N, int K, int sam, int sbn, int scm) {
  return ggemm::pw::fits(N, K) && (int64_t)sam * ggemm::pw::kTM < ggemm::nt::kOob &&
         (int64_t)sbn * ggemm::pw::kTN < ggemm::nt::kOob && (int64_t)scm * 2 * ggemm::pw::kTM < ggemm::nt::kOob;
}

// The automatic choice: the wide kernel wherever it fits. Against the 512-thread kernel it measured
// faster at all four fwd / dgrad sites on both row layouts: on the reference's contiguous K = 2880
// rows (half the 128-byte row segments straddle two lines) 2-6 % (5.690 against 5.999 ms over the
// four sites, same box), on line-aligned rows more.
bool wide_preferred(int N, int K, int sam, int sbn, int scm) { return wide_fits(N, K, sam, sbn, scm); }

int launch(const void* a, const void* b, void* out, const float* a_scale, const float* b_scale,
           const int64_t* group_offs, int G, int N, int K, int sam, int sbg, int sbn, int scm, int scn, int fmt,
           int64_t M_total, int kernel, void* stream) {
  int rc = validate(a, b, out, a_scale, b_scale, group_offs, G, N, K, sam, sbg, sbn, scm, scn, fmt, M_total);
  if (rc) return rc;
  const bool fits = wide_fits(N, K, sam, sbn, scm);
  if (kernel == GGEMM_PERSISTENT_KERNEL_WIDE && !fits) return GGEMM_E_SHAPE;
  if (kernel == GGEMM_PERSISTENT_KERNEL_AUTO)
    kernel = wide_preferred(N, K, sam, sbn, scm) ? GGEMM_PERSISTENT_KERNEL_WIDE : GGEMM_PERSISTENT_KERNEL_512;
  if (kernel < GGEMM_PERSISTENT_KERNEL_AUTO || kernel > GGEMM_PERSISTENT_KERNEL_WIDE) return GGEMM_E_SHAPE;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  if (M_total == 0) return GGEMM_OK;   // no rows: nothing to write
  const bool e5m2 = fmt == GGEMM_FP8_E5M2;
  if (kernel == GGEMM_PERSISTENT_KERNEL_WIDE) {
    auto kern = e5m2 ? _grouped_fp8_persistent_gemm_kernel_wide_e5m2 : _grouped_fp8_persistent_gemm_kernel_wide;
    hipLaunchKernelGGL(kern, dim3(cus), dim3(ggemm::pw::kNT), 0, (hipStream_t)stream, (const uint8_t*)a,
                       (const uint8_t*)b, (uint16_t*)out, a_scale, b_scale, group_offs, G, N, K, sam, sbg, sbn, scm,
                       scn, (void*)nullptr, (void*)nullptr, M_total);
    return (int)hipGetLastError();
  }
  auto kern = e5m2 ? _grouped_fp8_persistent_gemm_kernel_e5m2 : _grouped_fp8_persistent_gemm_kernel;
  hipLaunchKernelGGL(kern, dim3(cus), dim3(ggemm::kThreads), ggemm::kDynLdsBytes, (hipStream_t)stream,
                     (const uint8_t*)a, (const uint8_t*)b, (uint16_t*)out, a_scale, b_scale, group_offs, G, N, K, sam,
                     sbg, sbn, scm, scn, (void*)nullptr, (void*)nullptr, M_total);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

int ggemm_persistent_fp8(const void* a, const void* b, void* out, const float* a_scale, const float* b_scale,
                         const int64_t* group_offs, int32_t G, int32_t N, int32_t K, int32_t stride_am,
                         int32_t stride_bg, int32_t stride_bn, int32_t stride_cm, int32_t stride_cn,
                         int32_t a_format, int64_t M_total, void* stream) {
  return launch(a, b, out, a_scale, b_scale, group_offs, G, N, K, stride_am, stride_bg, stride_bn, stride_cm,
                stride_cn, a_format, M_total, GGEMM_PERSISTENT_KERNEL_AUTO, stream);
}

int ggemm_persistent_fp8_kernel(const void* a, const void* b, void* out, const float* a_scale, const float* b_scale,
                                const int64_t* group_offs, int32_t G, int32_t N, int32_t K, int32_t stride_am,
                                int32_t stride_bg, int32_t stride_bn, int32_t stride_cm, int32_t stride_cn,
                                int32_t a_format, int64_t M_total, int32_t kernel, void* stream) {
  return launch(a, b, out, a_scale, b_scale, group_offs, G, N, K, stride_am, stride_bg, stride_bn, stride_cm,
                stride_cn, a_format, M_total, kernel, stream);
}

int32_t ggemm_persistent_selected_kernel(int32_t N, int32_t K, int32_t stride_am, int32_t stride_bn,
                                         int32_t stride_cm) {
  return wide_preferred(N, K, stride_am, stride_bn, stride_cm) ? GGEMM_PERSISTENT_KERNEL_WIDE
                                                               : GGEMM_PERSISTENT_KERNEL_512;
}

int ggemm_persistent_clear_tail(void* out, int32_t N, int32_t stride_cm, const int64_t* group_offs, int32_t G,
                                int64_t M_total, void* stream) {
  if (!out || !group_offs) return GGEMM_E_NULL;
  if (G <= 0 || G > ggemm::nt::kMaxGroups || N <= 0 || N % 16 || M_total < 0 || M_total > ggemm::nt::kMaxRow)
    return GGEMM_E_SHAPE;
  if (stride_cm < N || stride_cm % 8) return GGEMM_E_STRIDE;
  if (!aligned(out, 16)) return GGEMM_E_ALIGN;
  int cus = 0;
  const int rc = device_cus(&cus);
  if (rc) return rc;
  if (M_total == 0) return GGEMM_OK;
  hipLaunchKernelGGL(clear_tail_kernel, dim3(4 * cus), dim3(kTailThreads), 0, (hipStream_t)stream,
                     static_cast<uint16_t*>(out), (int64_t)stride_cm, N, group_offs, G, M_total);
  return (int)hipGetLastError();
}

int ggemm_persistent_transpose_u8(const void* src, int32_t batch, int32_t rows, int32_t cols, int64_t src_bstride,
                                  int64_t src_rstride, void* dst, int64_t dst_bstride, int64_t dst_rstride,
                                  void* stream) {
  if (!src || !dst) return GGEMM_E_NULL;
  if (batch < 0 || rows <= 0 || cols <= 0 || rows % 16 || cols % 16) return GGEMM_E_SHAPE;
  if (src_rstride < cols || dst_rstride < rows || src_rstride % 16 || dst_rstride % 16 || src_bstride % 16 ||
      dst_bstride % 16)
    return GGEMM_E_STRIDE;
  if (batch > 1 && (src_bstride < (int64_t)rows * src_rstride || dst_bstride < (int64_t)cols * dst_rstride))
    return GGEMM_E_STRIDE;
  const int64_t per = (int64_t)((rows + kXT - 1) / kXT) * ((cols + kXT - 1) / kXT);
  if ((int64_t)batch * per > 0x7fffffffLL) return GGEMM_E_SHAPE;
  if (!aligned(src, 16) || !aligned(dst, 16)) return GGEMM_E_ALIGN;
  if (batch == 0) return GGEMM_OK;
  int cus = 0;
  const int rc = device_cus(&cus);
  if (rc) return rc;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(transpose_u8_kernel),
                                                   kXThreads, 0) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  if (per_cu > 3) per_cu = 3;   // as the transposing quantizer: 3 per CU beats the 4 or more that fit
  const int64_t tiles = (int64_t)batch * per, cap = (int64_t)cus * per_cu;
  const int grid = (int)(tiles < cap ? tiles : cap);
  hipLaunchKernelGGL(transpose_u8_kernel, dim3(grid), dim3(kXThreads), 0, (hipStream_t)stream,
                     static_cast<const uint8_t*>(src), batch, rows, cols, src_bstride, src_rstride,
                     static_cast<uint8_t*>(dst), dst_bstride, dst_rstride);
  return (int)hipGetLastError();
}

}  // extern "C"
