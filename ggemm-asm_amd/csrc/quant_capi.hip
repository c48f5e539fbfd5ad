// extern "C" launchers of the FP8 quantization producer (include/ggemm_quant.h), part of
// libggemm_vark.so. Arguments are validated on the host; nothing is launched on a validation error.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/ggemm_persistent.h"
#include "../../include/ggemm_quant.h"
#include "capi_common.h"
#include "quant_kernel.h"

static_assert(GGEMM_QUANT_MAX_GROUPS == ggemm::qt::kMaxGroups, "header and kernel agree");

namespace {

using ggemm::host::aligned;
using ggemm::host::device_cus;
namespace qt = ggemm::qt;

int check_2d(const void* x, int in_dtype, int64_t rows, int cols, int64_t stride) {
  if (!x) return GGEMM_E_NULL;
  if (in_dtype != GGEMM_IN_BF16 && in_dtype != GGEMM_IN_F32) return GGEMM_E_FORMAT;
  if (rows < 0 || cols <= 0 || cols % 8) return GGEMM_E_SHAPE;
  if (stride < cols || stride % 8) return GGEMM_E_STRIDE;
  if (!aligned(x, 16)) return GGEMM_E_ALIGN;
  return GGEMM_OK;
}

// Workgroups per CU of the streaming kernels' grid-stride launches. Measured on bf16 inputs of
// 0.75 and 1.5 GB: the quantize pass is fastest at 4 (16 waves per CU; 8 and 16 are 11-19 % slower
// on the larger tensor, 3 and fewer slower still), the read-only amax pass at 5.
constexpr int kQuantPerCu = 4;
constexpr int kAmaxPerCu = 5;

int grid_for(int64_t chunks, int cus, int per_cu) {
  const int64_t want = (chunks + (int64_t)qt::kThreads * qt::kUnroll - 1) / ((int64_t)qt::kThreads * qt::kUnroll);
  const int64_t cap = (int64_t)cus * per_cu;
  return (int)(want < 1 ? 1 : (want > cap ? cap : want));
}

void launch_amax(const void* x, int in_dtype, int64_t rows, int cols, int64_t stride, float* amax, int cus,
                 hipStream_t s) {
  uint32_t* bits = reinterpret_cast<uint32_t*>(amax);
  hipLaunchKernelGGL(qt::amax_init, dim3(1), dim3(64), 0, s, bits);
  if (rows == 0) return;
  const int grid = grid_for(rows * (cols / 8), cus, kAmaxPerCu);
  if (in_dtype == GGEMM_IN_F32)
    hipLaunchKernelGGL(qt::amax_kernel<true>, dim3(grid), dim3(qt::kThreads), 0, s, x, rows, cols, stride, bits);
  else
    hipLaunchKernelGGL(qt::amax_kernel<false>, dim3(grid), dim3(qt::kThreads), 0, s, x, rows, cols, stride, bits);
}

// Arguments of the transposing quantizer (all but the amax / history pointers).
int check_transpose(const void* x, int in_dtype, int batch, int rows, int cols, int out_format, const void* out,
                    int64_t out_stride, const void* out_t, int64_t out_t_stride, const float* scale_out) {
  if (!x || !out_t || !scale_out) return GGEMM_E_NULL;
  if (in_dtype != GGEMM_IN_BF16 && in_dtype != GGEMM_IN_F32) return GGEMM_E_FORMAT;
  if (out_format != GGEMM_FP8_E4M3 && out_format != GGEMM_FP8_E5M2) return GGEMM_E_FORMAT;
  if (batch < 0 || rows <= 0 || cols <= 0 || rows % 16 || cols % 16) return GGEMM_E_SHAPE;
  if ((out && (out_stride < cols || out_stride % 16)) || out_t_stride < rows || out_t_stride % 16)
    return GGEMM_E_STRIDE;
  // tile index (batch * tiles per matrix) and per-matrix offsets fit the kernel's integer widths
  const int64_t per = (int64_t)((rows + qt::kTT - 1) / qt::kTT) * ((cols + qt::kTT - 1) / qt::kTT);
  if (per > 0x7fffffffLL) return GGEMM_E_SHAPE;
  if (!aligned(x, 16) || !aligned(out_t, 16) || (out && !aligned(out, 16)) || !aligned(scale_out, 4))
    return GGEMM_E_ALIGN;
  return GGEMM_OK;
}

// Persistent grid of the transposing quantizer over 128 x 128 tiles: at most kTransposePerCu
// workgroups per CU (fewer if fewer fit). Measured on the [32, 5760, 2880] weight: 3 per CU is 1 %
// faster than the 4 or more that fit, 2 per CU 9 % slower.
constexpr int kTransposePerCu = 3;

int transpose_grid(const void* kernel, int batch, int rows, int cols, int cus) {
  const int64_t tiles = (int64_t)batch * ((rows + qt::kTT - 1) / qt::kTT) * ((cols + qt::kTT - 1) / qt::kTT);
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, qt::kThreads, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  if (per_cu > kTransposePerCu) per_cu = kTransposePerCu;
  const int64_t cap = (int64_t)cus * per_cu;
  return (int)(tiles < 1 ? 1 : (tiles < cap ? tiles : cap));
}

}  // namespace

extern "C" {

int ggemm_quant_amax(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride, float* amax_out,
                     void* stream) {
  int rc = check_2d(x, in_dtype, rows, cols, stride);
  if (rc) return rc;
  if (!amax_out) return GGEMM_E_NULL;
  if (!aligned(amax_out, 4)) return GGEMM_E_ALIGN;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  launch_amax(x, in_dtype, rows, cols, stride, amax_out, cus, (hipStream_t)stream);
  return (int)hipGetLastError();
}

int ggemm_quant_fp8_tensorwise(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride,
                               int32_t out_format, void* out, int64_t out_stride, float* scale_out,
                               float* amax_out, void* stream) {
  int rc = check_2d(x, in_dtype, rows, cols, stride);
  if (rc) return rc;
  if (!out || !scale_out || !amax_out) return GGEMM_E_NULL;
  if (out_format != GGEMM_FP8_E4M3 && out_format != GGEMM_FP8_E5M2) return GGEMM_E_FORMAT;
  if (out_stride < cols || out_stride % 8) return GGEMM_E_STRIDE;
  if (!aligned(out, 8) || !aligned(scale_out, 4) || !aligned(amax_out, 4)) return GGEMM_E_ALIGN;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  launch_amax(x, in_dtype, rows, cols, stride, amax_out, cus, s);
  const int grid = grid_for(rows * (cols / 8), cus, kQuantPerCu);
  const uint32_t* bits = reinterpret_cast<const uint32_t*>(amax_out);
  uint8_t* o = static_cast<uint8_t*>(out);
  const bool f32 = in_dtype == GGEMM_IN_F32, e5 = out_format == GGEMM_FP8_E5M2;
  auto k = f32 ? (e5 ? qt::quant_tensorwise_kernel<true, true> : qt::quant_tensorwise_kernel<true, false>)
               : (e5 ? qt::quant_tensorwise_kernel<false, true> : qt::quant_tensorwise_kernel<false, false>);
  hipLaunchKernelGGL(k, dim3(grid), dim3(qt::kThreads), 0, s, x, rows, cols, stride, o, out_stride, bits, scale_out);
  return (int)hipGetLastError();
}

// The delayed quantizers' history argument: a host slot in [0, H), or (slot_dev != nullptr) a device
// slot that history_advance moves on before the pass.
static int check_history(const float* amax_history, int32_t history_len, int32_t slot, const int32_t* slot_dev) {
  if (!amax_history) return GGEMM_E_NULL;
  if (history_len < 1 || history_len > GGEMM_QUANT_MAX_HISTORY) return GGEMM_E_SHAPE;
  if (!slot_dev && (slot < 0 || slot >= history_len)) return GGEMM_E_SHAPE;
  if (!aligned(amax_history, 4) || (slot_dev && !aligned(slot_dev, 4))) return GGEMM_E_ALIGN;
  return GGEMM_OK;
}

// Clears the history entry this call records into: hist[slot], or the device slot's next entry.
static void history_start(float* hist, int32_t H, int32_t slot, int32_t* slot_dev, hipStream_t s) {
  if (slot_dev)
    hipLaunchKernelGGL(qt::history_advance, dim3(1), dim3(64), 0, s, hist, H, slot_dev);
  else
    hipLaunchKernelGGL(qt::amax_init, dim3(1), dim3(64), 0, s, reinterpret_cast<uint32_t*>(hist + slot));
}

static int tensorwise_delayed(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride,
                              int32_t out_format, void* out, int64_t out_stride, float* amax_history,
                              int32_t history_len, int32_t slot, int32_t* slot_dev, float* scale_out, void* stream) {
  int rc = check_2d(x, in_dtype, rows, cols, stride);
  if (rc) return rc;
  if (!out || !scale_out) return GGEMM_E_NULL;
  if (out_format != GGEMM_FP8_E4M3 && out_format != GGEMM_FP8_E5M2) return GGEMM_E_FORMAT;
  rc = check_history(amax_history, history_len, slot, slot_dev);
  if (rc) return rc;
  if (out_stride < cols || out_stride % 8) return GGEMM_E_STRIDE;
  if (!aligned(out, 8) || !aligned(scale_out, 4)) return GGEMM_E_ALIGN;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  history_start(amax_history, history_len, slot, slot_dev, s);
  const int grid = grid_for(rows * (cols / 8), cus, kQuantPerCu);
  const bool f32 = in_dtype == GGEMM_IN_F32, e5 = out_format == GGEMM_FP8_E5M2;
  auto k = f32 ? (e5 ? qt::quant_tensorwise_delayed_kernel<true, true> : qt::quant_tensorwise_delayed_kernel<true, false>)
               : (e5 ? qt::quant_tensorwise_delayed_kernel<false, true>
                     : qt::quant_tensorwise_delayed_kernel<false, false>);
  hipLaunchKernelGGL(k, dim3(grid), dim3(qt::kThreads), 0, s, x, rows, cols, stride, static_cast<uint8_t*>(out),
                     out_stride, amax_history, history_len, slot, (const int32_t*)slot_dev, scale_out);
  return (int)hipGetLastError();
}

static int transpose_delayed(const void* x, int32_t in_dtype, int32_t batch, int32_t rows, int32_t cols,
                             int32_t out_format, void* out, int64_t out_stride, void* out_t, int64_t out_t_stride,
                             float* amax_history, int32_t history_len, int32_t slot, int32_t* slot_dev,
                             float* scale_out, void* stream) {
  int rc = check_history(amax_history, history_len, slot, slot_dev);
  if (rc) return rc;
  rc = check_transpose(x, in_dtype, batch, rows, cols, out_format, out, out_stride, out_t, out_t_stride, scale_out);
  if (rc) return rc;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  history_start(amax_history, history_len, slot, slot_dev, s);
  const bool f32 = in_dtype == GGEMM_IN_F32, e5 = out_format == GGEMM_FP8_E5M2;
  auto k = f32 ? (e5 ? qt::quant_transpose_delayed_kernel<true, true> : qt::quant_transpose_delayed_kernel<true, false>)
               : (e5 ? qt::quant_transpose_delayed_kernel<false, true>
                     : qt::quant_transpose_delayed_kernel<false, false>);
  const int grid = transpose_grid(reinterpret_cast<const void*>(k), batch, rows, cols, cus);
  hipLaunchKernelGGL(k, dim3(grid), dim3(qt::kThreads), 0, s, x, batch, rows, cols, static_cast<uint8_t*>(out),
                     out_stride, static_cast<uint8_t*>(out_t), out_t_stride, amax_history, history_len, slot,
                     (const int32_t*)slot_dev, scale_out);
  return (int)hipGetLastError();
}

int ggemm_quant_fp8_tensorwise_delayed(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride,
                                       int32_t out_format, void* out, int64_t out_stride, float* amax_history,
                                       int32_t history_len, int32_t slot, float* scale_out, void* stream) {
  return tensorwise_delayed(x, in_dtype, rows, cols, stride, out_format, out, out_stride, amax_history, history_len,
                            slot, nullptr, scale_out, stream);
}

int ggemm_quant_fp8_tensorwise_delayed_dev(const void* x, int32_t in_dtype, int64_t rows, int32_t cols,
                                           int64_t stride, int32_t out_format, void* out, int64_t out_stride,
                                           float* amax_history, int32_t history_len, int32_t* slot,
                                           float* scale_out, void* stream) {
  if (!slot) return GGEMM_E_NULL;
  return tensorwise_delayed(x, in_dtype, rows, cols, stride, out_format, out, out_stride, amax_history, history_len,
                            0, slot, scale_out, stream);
}

int ggemm_quant_fp8_tensorwise_transpose(const void* x, int32_t in_dtype, int32_t batch, int32_t rows, int32_t cols,
                                         int32_t out_format, void* out, int64_t out_stride, void* out_t,
                                         int64_t out_t_stride, float* scale_out, float* amax_out, void* stream) {
  if (!amax_out) return GGEMM_E_NULL;
  int rc = check_transpose(x, in_dtype, batch, rows, cols, out_format, out, out_stride, out_t, out_t_stride, scale_out);
  if (rc) return rc;
  if (!aligned(amax_out, 4)) return GGEMM_E_ALIGN;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  hipStream_t s = (hipStream_t)stream;
  launch_amax(x, in_dtype, (int64_t)batch * rows, cols, cols, amax_out, cus, s);
  const bool f32 = in_dtype == GGEMM_IN_F32, e5 = out_format == GGEMM_FP8_E5M2;
  auto k = f32 ? (e5 ? qt::quant_transpose_kernel<true, true> : qt::quant_transpose_kernel<true, false>)
               : (e5 ? qt::quant_transpose_kernel<false, true> : qt::quant_transpose_kernel<false, false>);
  const int grid = transpose_grid(reinterpret_cast<const void*>(k), batch, rows, cols, cus);
  hipLaunchKernelGGL(k, dim3(grid), dim3(qt::kThreads), 0, s, x, batch, rows, cols, static_cast<uint8_t*>(out),
                     out_stride, static_cast<uint8_t*>(out_t), out_t_stride,
                     reinterpret_cast<const uint32_t*>(amax_out), scale_out);
  return (int)hipGetLastError();
}

int ggemm_quant_fp8_tensorwise_transpose_delayed(const void* x, int32_t in_dtype, int32_t batch, int32_t rows,
                                                 int32_t cols, int32_t out_format, void* out, int64_t out_stride,
                                                 void* out_t, int64_t out_t_stride, float* amax_history,
                                                 int32_t history_len, int32_t slot, float* scale_out, void* stream) {
  return transpose_delayed(x, in_dtype, batch, rows, cols, out_format, out, out_stride, out_t, out_t_stride,
                           amax_history, history_len, slot, nullptr, scale_out, stream);
}

int ggemm_quant_fp8_tensorwise_transpose_delayed_dev(const void* x, int32_t in_dtype, int32_t batch, int32_t rows,
                                                     int32_t cols, int32_t out_format, void* out, int64_t out_stride,
                                                     void* out_t, int64_t out_t_stride, float* amax_history,
                                                     int32_t history_len, int32_t* slot, float* scale_out,
                                                     void* stream) {
  if (!slot) return GGEMM_E_NULL;
  return transpose_delayed(x, in_dtype, batch, rows, cols, out_format, out, out_stride, out_t, out_t_stride,
                           amax_history, history_len, 0, slot, scale_out, stream);
}

int ggemm_quant_mxfp8_grouped(const void* x, int32_t in_dtype, int64_t rows, int32_t cols, int64_t stride,
                              const int64_t* group_offs, int32_t G, int32_t out_format, void* out,
                              int64_t out_stride, int64_t out_rows, uint8_t* scales, int64_t scale_stride,
                              int64_t* padded_offs, void* stream) {
  int rc = check_2d(x, in_dtype, rows, cols, stride);
  if (rc) return rc;
  if (!group_offs || !out || !scales || !padded_offs) return GGEMM_E_NULL;
  if (out_format != GGEMM_FP8_E4M3 && out_format != GGEMM_FP8_E5M2) return GGEMM_E_FORMAT;
  if (G <= 0 || G > qt::kMaxGroups || cols % 16) return GGEMM_E_SHAPE;
  // 32-bit row indices inside the kernel
  if (rows + 31 * (int64_t)G > 0x7fffffffLL) return GGEMM_E_SHAPE;
  if (out_rows < rows + 31 * (int64_t)G) return GGEMM_E_SHAPE;
  if (out_stride < cols || out_stride % 16 || scale_stride < cols || scale_stride % 16) return GGEMM_E_STRIDE;
  if (!aligned(out, 16) || !aligned(scales, 16) || !aligned(padded_offs, 8) || !aligned(group_offs, 8))
    return GGEMM_E_ALIGN;
  int cus = 0;
  rc = device_cus(&cus);
  if (rc) return rc;
  qt::MxArgs a{x, rows, stride, cols, group_offs, G, static_cast<uint8_t*>(out), out_stride, scales, scale_stride,
               padded_offs};
  const bool f32 = in_dtype == GGEMM_IN_F32, e5 = out_format == GGEMM_FP8_E5M2;
  auto k = f32 ? (e5 ? qt::quant_mx_grouped_kernel<true, true> : qt::quant_mx_grouped_kernel<true, false>)
               : (e5 ? qt::quant_mx_grouped_kernel<false, true> : qt::quant_mx_grouped_kernel<false, false>);
  // persistent grid: workgroups that are resident together (the work is split statically, so a
  // workgroup that waits for a free slot would run its share afterwards), at most kMxPerCu per CU
  // (on dy bf16 [131072, 5760]: 2 per CU 1 % faster than the 4 or more that fit)
  constexpr int kMxPerCu = 2;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(k), qt::kThreads, 0) !=
          hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  if (per_cu > kMxPerCu) per_cu = kMxPerCu;
  hipLaunchKernelGGL(k, dim3(cus * per_cu), dim3(qt::kThreads), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
