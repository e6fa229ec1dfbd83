// transpose_f32: out[c * rows + r] = in[r * cols + c], bit-exact copy.
//
// Reference: operatorlib::transpose_f32 (src/transpose.cu:38-47) with a
// 32x33 padded shared tile and 32x8 thread blocks sized for 32-lane warps.
//
// MI355X design, two kernels:
//   * transpose_vec4_kernel (rows and cols multiples of 4, 16-byte aligned
//     buffers): a 128x128 fp32 tile per 512-thread workgroup, moved with
//     16-byte loads and stores in both directions. The 64 KiB tile sits in
//     LDS with a 129-float pitch; a wavefront's float4 writes (4 rows x 16
//     float4) and its 4-row column gathers for the output float4s hit
//     distinct banks. Long 512-byte row segments on both sides keep HBM
//     streaming at full rate.
//   * transpose_vec4u_kernel (any other shape or alignment of at least 64
//     such tiles, e.g. 4095x4097): the same 128x128 tiles with 16-byte
//     accesses at 4-byte alignment, float4s crossing the matrix edge moved
//     element by element, and cache hints chosen by which side is
//     misaligned (see vec4u_tile). Measured on MI355X against the 4-byte
//     kernel below (us, both hints non-temporal): 4095x4097 42.3 -> 36.6,
//     4097x4095 35.9 -> 33.9, 4096x4096 one element off alignment 41.1 ->
//     36.0, 8191x8193 157.3 -> 142.5.
//   * transpose_tile_kernel (smaller grids of any shape / alignment): a
//     64x64 tile per 512-thread workgroup (8 wavefronts, 8 rows each)
//     through a 64x65 LDS array; a wavefront reads one 256-byte input row
//     segment per load and writes one 256-byte output row segment per store.
//     The 65-float pitch puts element (r, c) in bank (r + c) mod 64, so both
//     the row-wise LDS writes and the column-wise reads are conflict-free.
// Interior tiles skip all bounds checks; edge tiles mask (per float4 in the
// vector kernel, where rows and cols are multiples of 4).
// The float4 kernel loads and stores non-temporally (each element is read
// and written once): 4.86 -> 5.17 TB/s at 4096 x 4096 with inputs cycling
// through 1 GiB. The same hints slowed the 4-byte kernel (4095 x 4097:
// 3.14 -> 2.81 TB/s), which keeps ordinary accesses.
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

typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kVecTile = 128;
constexpr int kVecPitch = kVecTile + 1;
constexpr int kVecPerThread = kVecTile * kVecTile / 4 / kThreads;  // 8

// One 128x128 tile; kFull drops the per-float4 bounds tests (interior
// tiles), so the full-tile path has no divergent branches.
template <bool kFull>
__device__ __forceinline__ void vec4_tile(const float* __restrict__ input,
                                          float* __restrict__ output, int rows,
                                          int cols, int row0, int col0,
                                          float* tile) {
  constexpr int kRowChunks = kVecTile / 4;  // float4s per tile row
  float4v v[kVecPerThread];
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const int q = static_cast<int>(threadIdx.x) + kThreads * i;
    const int r = q / kRowChunks;
    const int c = 4 * (q % kRowChunks);
    if (kFull || (row0 + r < rows && col0 + c < cols))
      v[i] = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(
          input + static_cast<std::size_t>(row0 + r) * cols + col0 + c));
  }
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const int q = static_cast<int>(threadIdx.x) + kThreads * i;
    float* d = tile + (q / kRowChunks) * kVecPitch + 4 * (q % kRowChunks);
    d[0] = v[i][0];
    d[1] = v[i][1];
    d[2] = v[i][2];
    d[3] = v[i][3];
  }
  __syncthreads();
  // Output tile row `orow` (= input column col0 + orow), float4 `oc`
  // (= input rows row0 + 4 oc .. + 3).
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const int q = static_cast<int>(threadIdx.x) + kThreads * i;
    const int orow = q / kRowChunks;
    const int oc = q % kRowChunks;
    if (kFull || (col0 + orow < cols && row0 + 4 * oc < rows)) {
      const float* s = tile + 4 * oc * kVecPitch + orow;
      const float4v q = {s[0], s[kVecPitch], s[2 * kVecPitch], s[3 * kVecPitch]};
      __builtin_nontemporal_store(
          q, reinterpret_cast<float4v*>(output + static_cast<std::size_t>(col0 + orow) * rows +
                                        row0 + 4 * oc));
    }
  }
}

__global__ __launch_bounds__(kThreads) void transpose_vec4_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows,
    int cols, int tiles_x, long long tiles) {
  __shared__ float tile[kVecTile * kVecPitch];
  for (long long t = blockIdx.x; t < tiles; t += gridDim.x) {
    int ty, tx;  // 32-bit division whenever the tile count allows
    if (tiles <= 0x7fffffffLL) {
      ty = static_cast<int>(t) / tiles_x;
      tx = static_cast<int>(t) - ty * tiles_x;
    } else {
      ty = static_cast<int>(t / tiles_x);
      tx = static_cast<int>(t % tiles_x);
    }
    const int row0 = ty * kVecTile;
    const int col0 = tx * kVecTile;
    if (row0 + kVecTile <= rows && col0 + kVecTile <= cols)
      vec4_tile<true>(input, output, rows, cols, row0, col0, tile);
    else
      vec4_tile<false>(input, output, rows, cols, row0, col0, tile);
    if (t + gridDim.x < tiles) __syncthreads();  // tile is rewritten next
  }
}

// Any shape and 4-byte alignment: the 128x128 tile kernel with dword-aligned
// 16-byte accesses (global_load/store_dwordx4 at any 4-byte phase, which the
// target's unaligned access mode allows). A float4 that crosses the matrix
// edge moves element by element.
typedef float float4u __attribute__((ext_vector_type(4), aligned(4)));
// Below this many 128x128 tiles the 4-byte 64x64 kernel is faster (its edge
// handling is lighter): 129x257 3.2 vs 4.7 us, 1000x1000 equal at 5.1 us.
constexpr long long kUnalignedMinTiles = 64;

// Cache hints per side. Measured on MI355X (us; non-temporal loads /
// stores vs the hints chosen here):
//   input rows misaligned only: 4096x4095 29.51 -> 28.03 (cached loads),
//     4096x4097 28.96 -> 27.53;
//   output rows misaligned only: 4095x4096 31.36 -> 30.30 (cached stores),
//     4097x4096 30.23 -> 29.87;
//   both: 4095x4097 36.70 -> 35.21 (cached loads, non-temporal stores;
//     cached stores as well: 37.10), 4097x4095 33.63 -> 31.93, 8191x8193
//     142.61 -> 134.29.
// Banding the tiles by XCD, so that tiles sharing a boundary line share an
// L2, cut FETCH_SIZE at 4095x4097 from 1.27x to 1.00x of the input bytes
// without changing the time (36.75 us): the misaligned 16-byte accesses
// themselves, not re-fetched lines, set the cost. Coalesced 4-byte stores
// for the misaligned output rows were slower (37.66 us).
template <bool kFull, bool kLoadNT, bool kStoreNT>
__device__ __forceinline__ void vec4u_tile(const float* __restrict__ input,
                                           float* __restrict__ output, int rows,
                                           int cols, int row0, int col0,
                                           float* tile) {
  constexpr int kRowChunks = kVecTile / 4;
  float4v v[kVecPerThread];
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const int q = static_cast<int>(threadIdx.x) + kThreads * i;
    const int r = row0 + q / kRowChunks;
    const int c = col0 + 4 * (q % kRowChunks);
    const float* src = input + static_cast<std::size_t>(r) * cols + c;
    if (kFull || (r < rows && c + 3 < cols)) {
      v[i] = kLoadNT ? __builtin_nontemporal_load(reinterpret_cast<const float4u*>(src))
                     : *reinterpret_cast<const float4u*>(src);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] = r < rows && c + j < cols ? src[j] : 0.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const int q = static_cast<int>(threadIdx.x) + kThreads * i;
    float* d = tile + (q / kRowChunks) * kVecPitch + 4 * (q % kRowChunks);
    d[0] = v[i][0];
    d[1] = v[i][1];
    d[2] = v[i][2];
    d[3] = v[i][3];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kVecPerThread; ++i) {
    const int q = static_cast<int>(threadIdx.x) + kThreads * i;
    const int orow = q / kRowChunks;
    const int oc = q % kRowChunks;
    const int c = col0 + orow;     // input column = output row
    const int r = row0 + 4 * oc;   // first of 4 input rows = output columns
    const float* s = tile + 4 * oc * kVecPitch + orow;
    float* dst = output + static_cast<std::size_t>(c) * rows + r;
    if (kFull || (c < cols && r + 3 < rows)) {
      const float4v o = {s[0], s[kVecPitch], s[2 * kVecPitch], s[3 * kVecPitch]};
      if (kStoreNT)
        __builtin_nontemporal_store(o, reinterpret_cast<float4u*>(dst));
      else
        *reinterpret_cast<float4u*>(dst) = o;
    } else if (c < cols) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (r + j < rows) dst[j] = s[j * kVecPitch];
    }
  }
}

template <bool kLoadNT, bool kStoreNT>
__global__ __launch_bounds__(kThreads) void transpose_vec4u_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows,
    int cols, int tiles_x, long long tiles) {
  __shared__ float tile[kVecTile * kVecPitch];
  for (long long t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int ty = static_cast<int>(t / tiles_x);
    const int tx = static_cast<int>(t % tiles_x);
    const int row0 = ty * kVecTile;
    const int col0 = tx * kVecTile;
    if (row0 + kVecTile <= rows && col0 + kVecTile <= cols)
      vec4u_tile<true, kLoadNT, kStoreNT>(input, output, rows, cols, row0, col0, tile);
    else
      vec4u_tile<false, kLoadNT, kStoreNT>(input, output, rows, cols, row0, col0, tile);
    if (t + gridDim.x < tiles) __syncthreads();  // tile is rewritten next
  }
}

}  // namespace

extern "C" int operatorlib_transpose_f32(const float* input, float* output,
                                         int rows, int cols,
                                         void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  hipStream_t stream = static_cast<hipStream_t>(stream_handle);
  constexpr long long kMaxGrid = 1LL << 30;
  if (rows % 4 == 0 && cols % 4 == 0 && opl::aligned16(input) &&
      opl::aligned16(output)) {
    const int tiles_x = (cols + kVecTile - 1) / kVecTile;
    const long long tiles =
        static_cast<long long>(tiles_x) * ((rows + kVecTile - 1) / kVecTile);
    const int blocks = static_cast<int>(tiles < kMaxGrid ? tiles : kMaxGrid);
    transpose_vec4_kernel<<<dim3(blocks), dim3(kThreads), 0, stream>>>(
        input, output, rows, cols, tiles_x, tiles);
    return hipGetLastError();
  }
  const int vtiles_x = (cols + kVecTile - 1) / kVecTile;
  const long long vtiles =
      static_cast<long long>(vtiles_x) * ((rows + kVecTile - 1) / kVecTile);
  if (vtiles >= kUnalignedMinTiles) {
    const int blocks = static_cast<int>(vtiles < kMaxGrid ? vtiles : kMaxGrid);
    const dim3 grid(blocks), block(kThreads);
    // Input rows are 16-byte aligned when cols % 4 == 0 and the input is;
    // output rows likewise with rows. This path has at least one side
    // misaligned.
    const bool in_aligned = cols % 4 == 0 && opl::aligned16(input);
    if (!in_aligned)
      transpose_vec4u_kernel<false, true><<<grid, block, 0, stream>>>(
          input, output, rows, cols, vtiles_x, vtiles);
    else  // only the output side is misaligned
      transpose_vec4u_kernel<true, false><<<grid, block, 0, stream>>>(
          input, output, rows, cols, vtiles_x, vtiles);
    return hipGetLastError();
  }
  const int tiles_x = (cols + kTile - 1) / kTile;
  const int tiles_y = (rows + kTile - 1) / kTile;
  const long long tiles = static_cast<long long>(tiles_x) * tiles_y;
  const int blocks = static_cast<int>(tiles < kMaxGrid ? tiles : kMaxGrid);
  transpose_tile_kernel<<<dim3(blocks), dim3(kThreads), 0, stream>>>(
      input, output, rows, cols, tiles_x, tiles);
  return hipGetLastError();
}
