// LDS tile map and register byte transpose shared by the two 128 x 128-tile transposes of
// libggemm_vark.so: the quantize-and-transpose producer (quant_kernel.h) and the byte transpose
// behind ggemm_persistent_transpose_u8 (persistent_capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ggemm {
namespace qt {

constexpr int kTT = 128;                    // transpose tile edge (elements)

// LDS tile of a transpose: 128 rows of 128 bytes, 16-byte chunk k of row r stored at
// chunk k ^ ((r >> 4) & 7). A thread's 16-byte write of a row chunk stays whole; the transposed
// read (the dword of 4 columns from 16 consecutive rows per thread, 8 threads per row group) finds
// the 8 row groups of a column group on 8 distinct chunk positions, i.e. distinct banks.
__device__ __forceinline__ int tt_off(int r, int c) {
  return r * kTT + ((((c >> 4) ^ (r >> 4)) & 7) << 4) + (c & 15);
}

// Bytes k of four dwords, packed low to high (one column of a 4 x 4 byte block).
__device__ __forceinline__ uint32_t byte_col(uint32_t a, uint32_t b, uint32_t c, uint32_t d, int k) {
  return ((a >> (8 * k)) & 0xffu) | (((b >> (8 * k)) & 0xffu) << 8) | (((c >> (8 * k)) & 0xffu) << 16) |
         (((d >> (8 * k)) & 0xffu) << 24);
}

}  // namespace qt
}  // namespace ggemm
