// FP8 quantization producer for the grouped GEMMs, gfx950 (MI355X, CDNA4): the step before the
// GEMMs, turning bf16 / fp32 activations, gradients and weights into their fp8 operands.
//
//  * amax:        amax = max |x| over a 2-D [rows, cols] tensor (NaN propagates).
//  * tensorwise:  scale = amax / fmax (1 when amax == 0), q = fp8(clamp(x / scale, -fmax, fmax));
//                 optionally with the transposed copy q^T of each matrix of a batch (weights).
//  * MX, grouped: groups of rows (the token axis) padded to multiples of 32 rows; per 32-row block
//                 and column, X = floor(log2(fl32(amax_blk / fmax))) clamped to [-127, 127]
//                 (0 for an all-zero block), e8m0 byte X + 127, q = fp8(clamp(x * 2^-X, +-fmax));
//                 padding rows are zero and the padded group offsets are written out.
//
// fmax = 448 (e4m3fn) or 57344 (e5m2). Rounding: x / scale is the correctly rounded fp32 quotient,
// fp32 -> fp8 is round-to-nearest-even (subnormals included), -0 keeps its sign, NaN becomes a NaN
// code of the format (0x7F or 0xFF: the sign of a NaN result is unspecified, as in IEEE
// arithmetic, and the GPU's x / NaN differs from a CPU's there). These are the recipes of the
// measured configurations (x / (amax/fmax) clamped and cast; MX block exponents from the block
// amax), with floor(log2()) taken exactly on the fp32 quotient.
//
// All three are HBM-bound streaming kernels: 16-byte (bf16) or 32-byte (fp32) loads of 8 elements
// per thread in the tensorwise path, 8-byte fp8 stores; the MX kernel keeps a 32-row x 4-column
// block in registers so x is read once. Every load and store of tensor data is non-temporal (it is
// touched once): with non-temporal fp8 stores the tensorwise pass moves its bytes about 12 % faster
// and the transposing pass about 10 % faster than with ordinary stores.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "transpose_tile.h"

namespace ggemm {
namespace qt {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;           // 16-byte chunks each thread has in flight in the streaming kernels
constexpr int kMaxGroups = 2047;     // MX: group offsets and padded offsets held in LDS

typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

template <bool kE5M2>
__device__ __forceinline__ constexpr float fmax_of() { return kE5M2 ? 57344.0f : 448.0f; }

// fp32 -> fp8 byte, round to nearest even. |f| <= fmax unless NaN (callers clamp first). The
// bit-level definition of the conversion; the kernels use the hardware instruction (pack4_fp8).
//  e4m3fn: bias 7, 3 mantissa bits, subnormals m * 2^-9; e5m2: bias 15, 2 bits, m * 2^-16.
// Normal range: add the rounding increment to the fp32 bits below the kept mantissa (a carry
// moves into the exponent, which is the correctly rounded result), then rebias. Subnormal range:
// |f| * 2^(9 or 16) is exact, and rint rounds half to even. Both are computed and the result is
// picked with bit masks: written as branches, the compiler emitted per-element exec-mask branches
// that cost more than the arithmetic.
template <bool kE5M2>
__device__ __forceinline__ uint32_t f32_to_fp8(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t s = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  constexpr int kMant = kE5M2 ? 2 : 3;
  constexpr int kShift = 23 - kMant;
  constexpr uint32_t kMinNormal = kE5M2 ? 0x38800000u : 0x3c800000u;   // 2^-14, 2^-6
  constexpr uint32_t kRebias = (kE5M2 ? (127 - 15) : (127 - 7)) << kMant;
  const uint32_t rn = ((a + ((1u << (kShift - 1)) - 1) + ((a >> kShift) & 1u)) >> kShift) - kRebias;
  // the subnormal candidate is only used for |f| < the smallest normal, where it is 0 .. 8 / 4
  const uint32_t rs = (uint32_t)__builtin_rintf(__uint_as_float(a < kMinNormal ? a : 0u) * (kE5M2 ? 65536.0f : 512.0f));
  const uint32_t normal = 0u - (uint32_t)(a >= kMinNormal);
  const uint32_t nan = 0u - (uint32_t)(a > 0x7f800000u);
  const uint32_t r = (rn & normal) | (rs & ~normal);
  return s | (r & ~nan) | (0x7fu & nan);
}

// Four clamped fp32 values -> four fp8 bytes (v[0] in the low byte) with the gfx950 conversion
// instruction, two values per instruction, rounding to nearest even. The GPU tests check it
// byte for byte against the bit-level definition above on every tie, both neighbours of each tie
// and fp32 subnormals.
template <bool kE5M2>
__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  if constexpr (kE5M2) {
    const int lo = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(c, d, lo, true);
  } else {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
  }
}

// clamp to [-fmax, fmax]; NaN stays NaN
template <bool kE5M2>
__device__ __forceinline__ float clamp_fmax(float v) {
  constexpr float m = fmax_of<kE5M2>();
  return v != v ? v : fminf(fmaxf(v, -m), m);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// 8 consecutive elements of row `row`, chunk `c` (elements 8c .. 8c+7), as fp32
template <bool kF32>
__device__ __forceinline__ void load8(const void* x, int64_t row, int64_t stride, int c, float v[8]) {
  if constexpr (kF32) {
    const v4f* p = (const v4f*)((const float*)x + row * stride + 8 * (int64_t)c);
    const v4f a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3]; v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
  } else {
    const v4u w = __builtin_nontemporal_load((const v4u*)((const uint16_t*)x + row * stride + 8 * (int64_t)c));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = bf16_lo(w[k]);
      v[2 * k + 1] = bf16_hi(w[k]);
    }
  }
}

// Row and 16-byte chunk of the kUnroll chunks a thread streams per round: flat chunk index
// i0 + u T (T = threads in the grid) split as (row, chunk) once, then advanced by kUnroll T per round
// with adds and one compare, instead of a 64-bit division per chunk.
struct ChunkWalk {
  int64_t row[kUnroll];
  int col[kUnroll];
  int64_t drow;
  int dcol, cpr;
  __device__ __forceinline__ ChunkWalk(int64_t i_first, int64_t T, int cpr_) : cpr(cpr_) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = i_first + u * T;
      row[u] = i / cpr;
      col[u] = (int)(i - row[u] * cpr);
    }
    const int64_t step = kUnroll * T;
    drow = step / cpr;
    dcol = (int)(step - drow * cpr);
  }
  __device__ __forceinline__ void advance() {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      col[u] += dcol;
      row[u] += drow;
      if (col[u] >= cpr) {
        col[u] -= cpr;
        ++row[u];
      }
    }
  }
};

// ---------------------------------------------------------------------------------- amax

__global__ void __launch_bounds__(64) amax_init(uint32_t* amax_bits) {
  if (threadIdx.x == 0) *amax_bits = 0u;
}

// Delayed scaling with the slot kept on the device: *slot (the previous call's slot) moves on to
// the next one, (slot + 1) mod H (a value outside [0, H) restarts at 0), and that entry is zeroed
// for this call's amax. Launched before the quantizing pass, which reads the slot back, so every
// launch -- a HIP graph replay included -- advances through the history.
__global__ void __launch_bounds__(64) history_advance(float* hist, int H, int32_t* slot) {
  if (threadIdx.x == 0) {
    const int32_t prev = *slot;
    const int32_t s = (prev >= 0 && prev < H - 1) ? prev + 1 : 0;
    *slot = s;
    reinterpret_cast<uint32_t*>(hist)[s] = 0u;
  }
}

// The workgroup's max of its threads' m (|x| as fp32 bits) into *amax_bits, one atomic.
__device__ __forceinline__ void block_amax(uint32_t m, uint32_t* amax_bits) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
  __shared__ uint32_t s_m[kThreads / 64];
  if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = max(m, s_m[w]);
    if (m) atomicMax(amax_bits, m);
  }
}

// max of |x| as fp32 bits (ordered like unsigned integers for non-negative values; any NaN is
// larger than +inf, so NaN propagates), one atomic per workgroup
template <bool kF32>
__global__ void __launch_bounds__(kThreads) amax_kernel(const void* x, int64_t rows, int cols, int64_t stride,
                                                        uint32_t* amax_bits) {
  const int cpr = cols / 8;
  const int64_t n = rows * cpr;
  const int64_t T = (int64_t)gridDim.x * kThreads;
  uint32_t m = 0;
  const int64_t i_first = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  ChunkWalk cw(i_first, T, cpr);
  // kUnroll chunks per thread and round: their loads are all in flight before the first is used
  for (int64_t i0 = i_first; i0 < n; i0 += kUnroll * T, cw.advance()) {
    float v[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (i0 + u * T < n) load8<kF32>(x, cw.row[u], stride, cw.col[u], v[u]);
      else for (int k = 0; k < 8; ++k) v[u][k] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int k = 0; k < 8; ++k) m = max(m, __float_as_uint(v[u][k]) & 0x7fffffffu);
  }
  block_amax(m, amax_bits);
}

// ---------------------------------------------------------------------------------- tensorwise

template <bool kE5M2>
__device__ __forceinline__ float tensor_scale(uint32_t amax_bits) {
  const float amax = __uint_as_float(amax_bits);
  return amax > 0.0f ? amax / fmax_of<kE5M2>() : (amax == 0.0f ? 1.0f : amax);   // NaN stays NaN
}

// x / scale, correctly rounded, computed as q = x y (y = fl(1 / scale)) corrected by one FMA
// residual: by Markstein's theorem fl(q + fl(x - q scale) y) is the correctly rounded quotient when y
// is the correctly rounded reciprocal and nothing over- or underflows. With amax finite and at least
// 2^-60 the scale and y are normal and |q| stays near fmax at most (|x| <= amax); an x small enough
// for the residual to underflow (|x| < 2^-102) has a quotient below 2^-26, which fp8 rounds to zero
// either way. Zero keeps the sign of x. Other amax (NaN, infinite, zero, below 2^-60) take the
// division itself, decided once per kernel (fast is uniform).
struct ScaleDiv {
  float scale, inv;
  bool fast;
};
template <bool kE5M2>
__device__ __forceinline__ ScaleDiv scale_div(uint32_t amax_bits) {
  const float amax = __uint_as_float(amax_bits);
  const float scale = tensor_scale<kE5M2>(amax_bits);
  return ScaleDiv{scale, 1.0f / scale, amax >= 0x1p-60f && amax <= 3.4028235e38f};   // false for NaN
}
// A scale that does not come from this tensor's amax (delayed scaling: earlier steps' amax). The
// FMA-corrected quotient (div_scale_guarded) is used for scales in [2^-80, 2^100]: the scale and
// its reciprocal are normal, a residual can underflow only for |x| < 2^-102, whose quotient is below
// 2^-22 and rounds to fp8 zero either way.
__device__ __forceinline__ ScaleDiv scale_div_given(float scale) {
  return ScaleDiv{scale, 1.0f / scale, scale >= 0x1p-80f && scale <= 0x1p100f};   // false for NaN
}

template <bool kFast>
__device__ __forceinline__ float div_scale(float x, const ScaleDiv& d) {
  if constexpr (kFast) {
    const float q = x * d.inv;
    const float r = __builtin_fmaf(-q, d.scale, x);
    const float c = __builtin_fmaf(r, d.inv, q);
    return __uint_as_float((__float_as_uint(c) & 0x7fffffffu) | (__float_as_uint(x) & 0x80000000u));
  } else {
    return x / d.scale;
  }
}

// x / scale when |x / scale| is not bounded by fmax (a given scale): a product x (1 / scale) beyond
// 2 fmax is returned as it is -- the exact quotient is then beyond fmax too and the clamp maps both
// to +-fmax -- so the correction never meets an overflow; below it the corrected quotient is the
// correctly rounded one (div_scale). NaN passes through.
template <bool kFast, bool kE5M2>
__device__ __forceinline__ float div_scale_guarded(float x, const ScaleDiv& d) {
  if constexpr (kFast) {
    const float q = x * d.inv;
    if (!(__builtin_fabsf(q) <= 2.0f * fmax_of<kE5M2>())) return q;
    return div_scale<true>(x, d);
  } else {
    return x / d.scale;
  }
}

template <bool kFast, bool kE5M2, bool kGiven>
__device__ __forceinline__ float quotient(float x, const ScaleDiv& d) {
  if constexpr (kGiven) return div_scale_guarded<kFast, kE5M2>(x, d);
  else return div_scale<kFast>(x, d);
}

// Largest |entry| (fp32 bits) of an amax history other than `slot`; NaN beats every number.
__device__ __forceinline__ uint32_t history_amax(const float* hist, int H, int slot) {
  uint32_t hm = 0;
  for (int i = 0; i < H; ++i)
    if (i != slot) hm = max(hm, __float_as_uint(hist[i]) & 0x7fffffffu);
  return hm;
}

// kGiven: the scale is a given one (guarded quotients) and the thread's max |x| (fp32 bits) is
// returned for the tensor's amax; otherwise 0.
template <bool kF32, bool kE5M2, bool kFast, bool kGiven = false>
__device__ __forceinline__ uint32_t tensorwise_body(const void* x, int64_t rows, int cols, int64_t stride,
                                                    uint8_t* out, int64_t out_stride, const ScaleDiv& d) {
  uint32_t m = 0;
  const int cpr = cols / 8;
  const int64_t n = rows * cpr;
  const int64_t T = (int64_t)gridDim.x * kThreads;
  const int64_t i_first = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  ChunkWalk cw(i_first, T, cpr);
  for (int64_t i0 = i_first; i0 < n; i0 += kUnroll * T, cw.advance()) {
    float v[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (i0 + u * T < n) load8<kF32>(x, cw.row[u], stride, cw.col[u], v[u]);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (i0 + u * T >= n) break;
      float y[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if constexpr (kGiven) {
          m = max(m, __float_as_uint(v[u][k]) & 0x7fffffffu);
          y[k] = clamp_fmax<kE5M2>(div_scale_guarded<kFast, kE5M2>(v[u][k], d));
        } else {
          y[k] = clamp_fmax<kE5M2>(div_scale<kFast>(v[u][k], d));
        }
      }
      const uint32_t w0 = pack4_fp8<kE5M2>(y[0], y[1], y[2], y[3]);
      const uint32_t w1 = pack4_fp8<kE5M2>(y[4], y[5], y[6], y[7]);
      __builtin_nontemporal_store(v2u{w0, w1}, (v2u*)(out + cw.row[u] * out_stride + 8 * (int64_t)cw.col[u]));
    }
  }
  return m;
}

template <bool kF32, bool kE5M2>
__global__ void __launch_bounds__(kThreads) quant_tensorwise_kernel(const void* x, int64_t rows, int cols,
                                                                    int64_t stride, uint8_t* out,
                                                                    int64_t out_stride, const uint32_t* amax_bits,
                                                                    float* scale_out) {
  const ScaleDiv d = scale_div<kE5M2>(*amax_bits);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = d.scale;
  if (d.fast)
    tensorwise_body<kF32, kE5M2, true>(x, rows, cols, stride, out, out_stride, d);
  else
    tensorwise_body<kF32, kE5M2, false>(x, rows, cols, stride, out, out_stride, d);
}

// Delayed scaling: scale = amax / fmax from the history's entries other than `slot` (the one this
// call replaces; 1 when they are all zero, NaN when one is NaN), written to scale_out; x quantized
// with it; the max |x| of this x reduced into hist[slot], which the host zeroed just before.
// slot_dev != nullptr: the slot is *slot_dev (set by history_advance just before) instead.
template <bool kF32, bool kE5M2>
__global__ void __launch_bounds__(kThreads) quant_tensorwise_delayed_kernel(const void* x, int64_t rows, int cols,
                                                                            int64_t stride, uint8_t* out,
                                                                            int64_t out_stride, float* hist, int H,
                                                                            int slot, const int32_t* slot_dev,
                                                                            float* scale_out) {
  if (slot_dev) slot = *slot_dev;
  const ScaleDiv d = scale_div_given(tensor_scale<kE5M2>(history_amax(hist, H, slot)));
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = d.scale;
  const uint32_t m = d.fast ? tensorwise_body<kF32, kE5M2, true, true>(x, rows, cols, stride, out, out_stride, d)
                            : tensorwise_body<kF32, kE5M2, false, true>(x, rows, cols, stride, out, out_stride, d);
  block_amax(m, reinterpret_cast<uint32_t*>(hist + slot));
}

// ---------------------------------------------------------------------------------- tensorwise + transpose

// Per-tensor quantization of a batch of [rows, cols] matrices (contiguous x [batch, rows, cols])
// writing q^T [batch, cols, rows] (row stride out_t_stride bytes) and, when out != nullptr, q
// [batch, rows, cols] (row stride out_stride bytes; padded strides keep rows line-aligned): a weight [G, N, K]
// quantized once for both the forward GEMM (B = w, K-major) and the data-gradient GEMM (B = w^T,
// N-major). rows and cols are multiples of 16. Persistent grid over 128 x 128 tiles, so every row
// segment of q and of q^T a tile writes is one whole 128-byte line: thread t quantizes 16 elements
// of each of the tile rows t / 8 + 32h (h = 0..3; all four loads issued before any is used), writes
// its bytes of q and deposits them in an LDS tile (tt_off); after a barrier it reads the dwords of
// tile columns 4 (t / 8) .. +3 in tile rows 16 (t % 8) .. +15 and writes 16 bytes to each of those
// four q^T rows, so the 8 threads of a column group cover one 128-byte line per store instruction.
// The 16-element segments of a ragged edge tile are wholly inside the matrix or outside.

// kGiven as in tensorwise_body: guarded quotients, and the thread's max |x| returned.
template <bool kF32, bool kE5M2, bool kFast, bool kGiven = false>
__device__ __forceinline__ uint32_t transpose_body(const void* x, int batch, int rows, int cols, uint8_t* out,
                                                   int64_t out_stride, uint8_t* out_t, int64_t out_t_stride,
                                                   const ScaleDiv& d, uint8_t* s_t) {
  uint32_t m = 0;
  const int tid = threadIdx.x;
  const int tr = tid >> 3;                  // first tile row (then + 32, + 64, + 96)
  const int tc = 16 * (tid & 7);            // first tile column of this thread's segments
  const int cg = tid >> 3;                  // q^T: tile columns 4 cg .. 4 cg + 3 (rows of q^T)
  const int rj = tid & 7;                   // q^T: tile rows 16 rj .. 16 rj + 15 (8 threads: one line)
  const int rt = (rows + kTT - 1) / kTT, ct = (cols + kTT - 1) / kTT;
  const int per = rt * ct;
  const int64_t tiles = (int64_t)batch * per;
  for (int64_t it = blockIdx.x; it < tiles; it += gridDim.x) {
    const int b = (int)(it / per);
    const int rem = (int)(it - (int64_t)b * per);
    const int r0 = (rem / ct) * kTT, c0 = (rem % ct) * kTT;
    const bool col_in = c0 + tc < cols;
    float v[4][16];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int64_t row = (int64_t)b * rows + r0 + tr + 32 * h;
      if (col_in && r0 + tr + 32 * h < rows) {
        load8<kF32>(x, row, cols, (c0 + tc) / 8, v[h]);
        load8<kF32>(x, row, cols, (c0 + tc) / 8 + 1, v[h] + 8);
      }
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      if (!(col_in && r0 + tr + 32 * h < rows)) continue;
      if constexpr (kGiven) {
#pragma unroll
        for (int k = 0; k < 16; ++k) m = max(m, __float_as_uint(v[h][k]) & 0x7fffffffu);
      }
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = pack4_fp8<kE5M2>(clamp_fmax<kE5M2>(quotient<kFast, kE5M2, kGiven>(v[h][4 * k], d)),
                                clamp_fmax<kE5M2>(quotient<kFast, kE5M2, kGiven>(v[h][4 * k + 1], d)),
                                clamp_fmax<kE5M2>(quotient<kFast, kE5M2, kGiven>(v[h][4 * k + 2], d)),
                                clamp_fmax<kE5M2>(quotient<kFast, kE5M2, kGiven>(v[h][4 * k + 3], d)));
      const int64_t row = (int64_t)b * rows + r0 + tr + 32 * h;
      if (out) __builtin_nontemporal_store(v4u{w[0], w[1], w[2], w[3]}, (v4u*)(out + row * out_stride + c0 + tc));
      *(v4u*)(s_t + tt_off(tr + 32 * h, tc)) = v4u{w[0], w[1], w[2], w[3]};
    }
    __syncthreads();
    // q^T: the dwords of columns 4 cg .. 4 cg + 3 in rows 16 rj + i, transposed in registers into
    // 16 bytes of each of the four q^T rows; a store instruction's 8 threads of a row group write
    // one whole 128-byte line
    if (r0 + 16 * rj < rows && c0 + 4 * cg < cols) {
      uint32_t dw[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) dw[i] = *(const uint32_t*)(s_t + tt_off(16 * rj + i, 4 * cg));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        uint8_t* dst = out_t + ((int64_t)b * cols + c0 + 4 * cg + k) * out_t_stride + r0 + 16 * rj;
        __builtin_nontemporal_store(v4u{byte_col(dw[0], dw[1], dw[2], dw[3], k), byte_col(dw[4], dw[5], dw[6], dw[7], k),
                                        byte_col(dw[8], dw[9], dw[10], dw[11], k),
                                        byte_col(dw[12], dw[13], dw[14], dw[15], k)},
                                    (v4u*)dst);
      }
    }
    __syncthreads();
  }
  return m;
}

template <bool kF32, bool kE5M2>
__global__ void __launch_bounds__(kThreads) quant_transpose_kernel(const void* x, int batch, int rows, int cols,
                                                                   uint8_t* out, int64_t out_stride, uint8_t* out_t,
                                                                   int64_t out_t_stride, const uint32_t* amax_bits,
                                                                   float* scale_out) {
  __shared__ __attribute__((aligned(16))) uint8_t s_t[kTT * kTT];
  const ScaleDiv d = scale_div<kE5M2>(*amax_bits);
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = d.scale;
  if (d.fast)
    transpose_body<kF32, kE5M2, true>(x, batch, rows, cols, out, out_stride, out_t, out_t_stride, d, s_t);
  else
    transpose_body<kF32, kE5M2, false>(x, batch, rows, cols, out, out_stride, out_t, out_t_stride, d, s_t);
}

// Delayed scaling of the transposing pass: the scale from the history's entries other than `slot`
// (as quant_tensorwise_delayed_kernel), the max |x| of this x reduced into hist[slot], which the
// host zeroed just before; slot_dev as in quant_tensorwise_delayed_kernel.
template <bool kF32, bool kE5M2>
__global__ void __launch_bounds__(kThreads) quant_transpose_delayed_kernel(const void* x, int batch, int rows,
                                                                           int cols, uint8_t* out, int64_t out_stride,
                                                                           uint8_t* out_t, int64_t out_t_stride,
                                                                           float* hist, int H, int slot,
                                                                           const int32_t* slot_dev, float* scale_out) {
  __shared__ __attribute__((aligned(16))) uint8_t s_t[kTT * kTT];
  if (slot_dev) slot = *slot_dev;
  const ScaleDiv d = scale_div_given(tensor_scale<kE5M2>(history_amax(hist, H, slot)));
  if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = d.scale;
  const uint32_t m =
      d.fast ? transpose_body<kF32, kE5M2, true, true>(x, batch, rows, cols, out, out_stride, out_t, out_t_stride, d, s_t)
             : transpose_body<kF32, kE5M2, false, true>(x, batch, rows, cols, out, out_stride, out_t, out_t_stride, d,
                                                        s_t);
  block_amax(m, reinterpret_cast<uint32_t*>(hist + slot));
}

// ---------------------------------------------------------------------------------- MX, grouped

// e8m0 exponent of a 32-row block column: floor(log2(fl32(amax / fmax))) clamped to [-127, 127],
// 0 for amax == 0; a NaN amax gives the e8m0 NaN code (returned as 128: byte 0xFF).
template <bool kE5M2>
__device__ __forceinline__ int block_exponent(float amax) {
  if (amax != amax) return 128;
  if (amax == 0.0f) return 0;
  const float y = amax / fmax_of<kE5M2>();
  if (y > 3.4028235e38f) return 127;                       // inf
  const int e = (int)(__float_as_uint(y) >> 23) - 127;   // the exponent field; a subnormal
  return e < -127 ? -127 : e;                              // quotient (field 0) is below 2^-126
}

struct MxArgs {
  const void* x;
  int64_t rows;
  int64_t stride;
  int cols;
  const int64_t* group_offs;
  int G;
  uint8_t* out;
  int64_t out_stride;
  uint8_t* scales;
  int64_t scale_stride;
  int64_t* padded_offs;
};

// Persistent grid. Prologue: group offsets and padded offsets (prefix sums of ceil(len/32)*32) in
// LDS; workgroup 0 writes the padded offsets. Work item = (32-row output block, 256 columns), one
// per wave: lane l owns columns 4l .. 4l+3, loads the block's 32 source rows (zeros for padding),
// reduces the column amax, and writes 32 rows of 4 fp8 bytes plus one row of 4 e8m0 bytes.
template <bool kF32, bool kE5M2>
__global__ void __launch_bounds__(kThreads) quant_mx_grouped_kernel(MxArgs a) {
  __shared__ int s_offs[kMaxGroups + 1];
  __shared__ int s_pad[kMaxGroups + 1];
  __shared__ int s_part[kThreads];
  __shared__ bool s_flag;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = a.G;
  {
    constexpr int kPer = (kMaxGroups + 1) / kThreads;     // 8 groups per thread
    int o[kPer + 1];
#pragma unroll
    for (int k = 0; k <= kPer; ++k) {
      const int64_t v = a.group_offs[min(tid * kPer + k, G)];
      o[k] = v < 0 ? -1 : (v > a.rows ? (int)min(a.rows + 1, (int64_t)0x7fffffff) : (int)v);
    }
    int mine[kPer], sum = 0;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int g = tid * kPer + k;
      const int len = g < G ? o[k + 1] - o[k] : 0;
      bad |= len < 0 || (g <= G && (o[k] < 0 || o[k] > a.rows));
      mine[k] = len > 0 ? (len + 31) / 32 * 32 : 0;
      sum += mine[k];
      if (g <= G) s_offs[g] = o[k];
    }
    // offsets outside [0, rows] or decreasing: nothing is read or written (the host checks the
    // output capacity against rows + 31 G, which holds only for valid offsets)
    s_part[tid] = bad ? -1 : sum;
    __syncthreads();
    if (tid == 0) {
      bool any = false;
      for (int t = 0; t < kThreads; ++t) any |= s_part[t] < 0;
      s_flag = any;
    }
    __syncthreads();
    if (s_flag) return;
    s_part[tid] = sum;
    __syncthreads();
    for (int d = 1; d < kThreads; d <<= 1) {
      const int v = tid >= d ? s_part[tid - d] : 0;
      __syncthreads();
      s_part[tid] += v;
      __syncthreads();
    }
    int run = s_part[tid] - sum;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int g = tid * kPer + k;
      if (g < G) s_pad[g] = run;
      run += mine[k];
    }
    if (tid == kThreads - 1) s_pad[G] = s_part[tid];
    __syncthreads();
  }
  if (blockIdx.x == 0)
    for (int g = tid; g <= G; g += kThreads) a.padded_offs[g] = s_pad[g];

  const int blocks = s_pad[G] / 32;
  const int strips = (a.cols + 255) / 256;
  const int64_t items = (int64_t)blocks * strips;
  const int col = 4 * lane;
  for (int64_t it = (int64_t)blockIdx.x * (kThreads / 64) + wave; it < items;
       it += (int64_t)gridDim.x * (kThreads / 64)) {
    const int b = (int)(it / strips);
    const int c0 = (int)(it - (int64_t)b * strips) * 256 + col;
    const int p0 = 32 * b;
    int lo = 0, hi = G - 1;                                // group: the last g with s_pad[g] <= p0
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_pad[mid] <= p0) lo = mid; else hi = mid - 1;
    }
    // wave-uniform: scalar registers, so the row guards below are scalar branches
    lo = __builtin_amdgcn_readfirstlane(lo);
    const int src0 = __builtin_amdgcn_readfirstlane(s_offs[lo] + (p0 - s_pad[lo]));   // row of padded p0
    const int valid = __builtin_amdgcn_readfirstlane(min(32, s_offs[lo + 1] - src0));  // >= 1 source rows
    if (c0 >= a.cols) continue;                            // lanes past the last column
    // The block's 32 rows x 4 columns stay in registers between the amax and the conversion:
    // fp32 as loaded, bf16 as loaded (two values per register; widened when used).
    constexpr int kW = kF32 ? 4 : 2;
    uint32_t r[32][kW];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (i < valid) {
        if constexpr (kF32) {
          const v4u t = __builtin_nontemporal_load((const v4u*)((const float*)a.x + (int64_t)(src0 + i) * a.stride + c0));
          r[i][0] = t[0]; r[i][1] = t[1]; r[i][2] = t[2]; r[i][3] = t[3];
        } else {
          const v2u t = __builtin_nontemporal_load((const v2u*)((const uint16_t*)a.x + (int64_t)(src0 + i) * a.stride + c0));
          r[i][0] = t[0]; r[i][1] = t[1];
        }
      } else {
#pragma unroll
        for (int k = 0; k < kW; ++k) r[i][k] = 0u;
      }
    }
    auto val = [&](int i, int j) -> float {
      if constexpr (kF32) return __uint_as_float(r[i][j]);
      else return (j & 1) ? bf16_hi(r[i][j >> 1]) : bf16_lo(r[i][j >> 1]);
    };
    uint32_t sc = 0;
    float mul[4];
    uint32_t am[4] = {0u, 0u, 0u, 0u};       // |x| bit patterns order like the values
    if constexpr (kF32) {
#pragma unroll
      for (int i = 0; i < 32; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) am[j] = max(am[j], r[i][j] & 0x7fffffffu);
    } else {
      // bf16 pairs: the amax runs on the 16-bit patterns, so nothing is widened before use
#pragma unroll
      for (int i = 0; i < 32; ++i)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          am[2 * k] = max(am[2 * k], r[i][k] & 0x7fffu);
          am[2 * k + 1] = max(am[2 * k + 1], (r[i][k] >> 16) & 0x7fffu);
        }
#pragma unroll
      for (int j = 0; j < 4; ++j) am[j] <<= 16;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int X = block_exponent<kE5M2>(__uint_as_float(am[j]));
      sc |= (uint32_t)(X + 127) << (8 * j);
      mul[j] = X == 128 ? __uint_as_float(0x7fc00000u) : __builtin_ldexpf(1.0f, -X);   // exact 2^-X
    }
    __builtin_nontemporal_store(sc, (uint32_t*)(a.scales + (int64_t)b * a.scale_stride + c0));
    uint8_t* orow = a.out + (int64_t)p0 * a.out_stride + c0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      __builtin_nontemporal_store(
          pack4_fp8<kE5M2>(clamp_fmax<kE5M2>(val(i, 0) * mul[0]), clamp_fmax<kE5M2>(val(i, 1) * mul[1]),
                           clamp_fmax<kE5M2>(val(i, 2) * mul[2]), clamp_fmax<kE5M2>(val(i, 3) * mul[3])),
          (uint32_t*)orow);
      orow += a.out_stride;
    }
  }
}

}  // namespace qt
}  // namespace ggemm
