// transpose_f32: out[c * rows + r] = in[r * cols + c], bit-exact copy.
//
// Reference: operatorlib::transpose_f32 (src/transpose.cu:38-47) with a
// 32x33 padded shared tile and 32x8 thread blocks sized for 32-lane warps.
//
// MI355X design, four tiled kernels, and two for thin matrices (at most 16
// rows or columns: transpose_thin4_kernel / transpose_thin_kernel, one
// thread per 4 or 1 indices of the long side; described before them):
//   * transpose_vec4_kernel (rows and cols multiples of 4, 16-byte aligned
//     buffers): a 128x128 fp32 tile per 512-thread workgroup, moved with
//     16-byte loads and stores in both directions. The 64 KiB tile sits in
//     LDS with a 129-float pitch; a wavefront's float4 writes (4 rows x 16
//     float4) and its 4-row column gathers for the output float4s hit
//     distinct banks. Tiles are taken in strips of 16 tile columns
//     (strip_tile), so the tiles resident together read and write rows in
//     runs of several KiB on both sides.
//   * transpose_window_kernel (output rows not 16-byte aligned, at least 64
//     128x128 tiles' worth, e.g. 4095x4097): aligned float4 windows on both
//     sides, each output row segment starting on a 64-byte boundary (described
//     before it).
//   * transpose_vec4u_kernel (only the input rows misaligned, e.g.
//     4096x4095): the 128x128 tiles with 16-byte accesses at 4-byte
//     alignment, float4s crossing the matrix edge moved element by element,
//     cached loads and non-temporal stores (see vec4u_tile). Measured on
//     MI355X against the 4-byte kernel below (us, both hints
//     non-temporal): 4095x4097 42.3 -> 36.6, 4097x4095 35.9 -> 33.9,
//     4096x4096 one element off alignment 41.1 -> 36.0, 8191x8193 157.3 ->
//     142.5.
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

// Thin matrices (at most kThinMax rows or columns): one thread per index of
// the long dimension, so a wavefront's lanes cover 256 contiguous bytes on
// that side per access, and the short side (s <= S elements, in registers)
// is looped over; its accesses are s floats apart, and the wavefront's s
// accesses together cover one contiguous range. The tiled kernels spent
// nearly whole tiles of padding here (1 x 2^20: 97.5 us, 2^20 x 3: 52 us,
// against a 3.7 us copy of the same bytes; 2^20 x 16: 51.6 us, 13 x 100003:
// 13.6 us, now 26.0 and 8.0). Loads are issued from clamped indices,
// unconditionally, so they leave back to back.
constexpr int kThinMax = 16;
constexpr int kThinThreads = 256;
constexpr int kThinMaxBlocks = 8192;

template <int S, bool kShortRows>
__global__ __launch_bounds__(kThinThreads) void transpose_thin_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows, int cols) {
  const int s = kShortRows ? rows : cols;
  const long long n = kShortRows ? cols : rows;
  for (long long i = static_cast<long long>(blockIdx.x) * kThinThreads + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * kThinThreads) {
    float v[S];
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const long long jj = j < s ? j : s - 1;
      v[j] = kShortRows ? input[jj * n + i] : input[i * s + jj];
    }
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < s) {
        if constexpr (kShortRows)
          output[i * s + j] = v[j];
        else
          output[static_cast<long long>(j) * n + i] = v[j];
      }
    }
  }
}

// The same for a long side that is a multiple of 4 with 16-byte aligned
// buffers: a thread moves 4 consecutive indices of the long side as S
// float4 loads and S float4 stores (the S x 4 block transposed in
// registers; S is exact, so every register index is a constant), instead
// of 4 S scalar accesses. The long side's accesses are contiguous per
// wavefront and non-temporal; the short side's (16 bytes every 16 S) are
// cached, so that L2 merges the partial lines.
typedef float float4t __attribute__((ext_vector_type(4)));

template <int S, bool kShortRows>
__global__ __launch_bounds__(kThinThreads) void transpose_thin4_kernel(
    const float* __restrict__ input, float* __restrict__ output, long long n) {
  const long long groups = n / 4;
  for (long long g = static_cast<long long>(blockIdx.x) * kThinThreads + threadIdx.x;
       g < groups; g += static_cast<long long>(gridDim.x) * kThinThreads) {
    const long long i0 = 4 * g;
    float v[4 * S];
    if constexpr (kShortRows) {
      // v[4 j + a] = input[j][i0 + a]; output row i0 + a holds v[4 j + a]
      // at column j, so its flat element e = a S + j
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const float4t q = __builtin_nontemporal_load(
            reinterpret_cast<const float4t*>(input + j * n + i0));
#pragma unroll
        for (int a = 0; a < 4; ++a) v[4 * j + a] = q[a];
      }
#pragma unroll
      for (int f = 0; f < S; ++f) {
        float4t o;
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = v[4 * ((4 * f + c) % S) + (4 * f + c) / S];
        // cached: a store instruction writes 16 of every 16 S bytes, and the
        // wavefront's S stores complete the lines in L2 (non-temporal partial
        // lines: 8 x 2^20 67 us against 25 for the scalar kernel)
        *reinterpret_cast<float4t*>(output + i0 * S + 4 * f) = o;
      }
    } else {
      // rows i0 .. i0 + 3 of S columns are 4 S consecutive floats: v[a S + j]
#pragma unroll
      for (int f = 0; f < S; ++f) {
        const float4t q = *reinterpret_cast<const float4t*>(input + i0 * S + 4 * f);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[4 * f + c] = q[c];
      }
#pragma unroll
      for (int j = 0; j < S; ++j) {
        float4t o;
#pragma unroll
        for (int a = 0; a < 4; ++a) o[a] = v[a * S + j];
        __builtin_nontemporal_store(o, reinterpret_cast<float4t*>(output + j * n + i0));
      }
    }
  }
}

template <bool kShortRows, int S = 1>
void launch_thin4(const float* input, float* output, int s, long long n, hipStream_t stream) {
  if constexpr (S < kThinMax) {
    if (s > S) return launch_thin4<kShortRows, S + 1>(input, output, s, n, stream);
  }
  const long long blocks = (n / 4 + kThinThreads - 1) / kThinThreads;
  transpose_thin4_kernel<S, kShortRows>
      <<<dim3(static_cast<unsigned>(blocks < kThinMaxBlocks ? blocks : kThinMaxBlocks)),
         dim3(kThinThreads), 0, stream>>>(input, output, n);
}

template <bool kShortRows, int S = 1>
void launch_thin(const float* input, float* output, int rows, int cols, hipStream_t stream) {
  const int s = kShortRows ? rows : cols;
  if constexpr (S < kThinMax) {
    if (s > S) return launch_thin<kShortRows, 2 * S>(input, output, rows, cols, stream);
  }
  const long long n = kShortRows ? cols : rows;
  const long long blocks = (n + kThinThreads - 1) / kThinThreads;
  transpose_thin_kernel<S, kShortRows>
      <<<dim3(static_cast<unsigned>(blocks < kThinMaxBlocks ? blocks : kThinMaxBlocks)),
         dim3(kThinThreads), 0, stream>>>(input, output, rows, cols);
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

// Tile order of transpose_vec4_kernel: strips of G = 16 tile columns,
// each walked top to bottom, G tiles across per tile row (the
// last strip as wide as the columns left). The ~512 tiles resident at a
// time (two workgroups per CU) then form a window about as tall as it is
// wide, so both the input rows read and the output rows written run in
// contiguous pieces of several KiB, where row-major tile order reads whole
// input rows but scatters every output row over 512-byte pieces. Measured
// on MI355X (us, row-major -> strips of 16; strips of 12 / 24 / 32 were
// no better overall): 4096^2 25.8 -> 24.5, 8192^2 96.8 -> 88.6, 12288^2
// 262.0 -> 224.0, 16384x4096 103.4 -> 95.4, 2048x16384 54.2 -> 50.9,
// 1024x8192 15.7 -> 14.5, 8192x4096 45.9 -> 45.4, 4096x4100 27.9 -> 27.1;
// within 1% either way at 2048^2, 8192x1024, 3000x5000 and 1000^2.
// transpose_vec4u_kernel takes strips of 8, measured best for it (see
// there).
// transpose_window_kernel keeps row-major order (strips of 16 to 48 were
// 2-7% slower at 4095x4097, 4097x4095 and 8191x8193).
template <int G, typename I>
__device__ __forceinline__ void strip_tile(I t, int tiles_x, I tiles_y, int* ty, int* tx) {
  const int full = tiles_x / G * G;  // columns in whole strips
  const I in_full = static_cast<I>(full) * tiles_y;
  if (t < in_full) {
    const I per_strip = static_cast<I>(G) * tiles_y;
    const I strip = t / per_strip;
    const I r = t - strip * per_strip;
    *ty = static_cast<int>(r / G);
    *tx = static_cast<int>(strip) * G + static_cast<int>(r % G);
  } else {
    const int w = tiles_x - full;
    const I r = t - in_full;
    *ty = static_cast<int>(r / w);
    *tx = full + static_cast<int>(r % w);
  }
}

__global__ __launch_bounds__(kThreads) void transpose_vec4_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows,
    int cols, int tiles_x, long long tiles) {
  __shared__ float tile[kVecTile * kVecPitch];
  const long long tiles_y = tiles / tiles_x;
  for (long long t = blockIdx.x; t < tiles; t += gridDim.x) {
    int ty, tx;  // 32-bit division whenever the tile count allows
    if (tiles <= 0x7fffffffLL)
      strip_tile<16, int>(static_cast<int>(t), tiles_x, static_cast<int>(tiles_y), &ty, &tx);
    else
      strip_tile<16, long long>(t, tiles_x, tiles_y, &ty, &tx);
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
// without changing the time (36.75 us): re-fetched input lines do not set
// the cost. Coalesced 4-byte stores for the misaligned output rows were
// slower (37.66 us). Output rows misaligned now go to
// transpose_window_kernel; this kernel keeps cached loads and
// non-temporal stores for the input-misaligned case.
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
  const long long tiles_y = tiles / tiles_x;
  for (long long t = blockIdx.x; t < tiles; t += gridDim.x) {
    // strips of 8 tile columns (strip_tile); measured on MI355X (us,
    // row-major -> strips of 8; 12, 16 and 24 were no better overall):
    // 4096x4095 28.0 -> 26.4, 4096x4097 27.2 -> 26.1, 8192x8191 105.3 ->
    // 94.2, 2048x6001 20.6 -> 20.5
    int ty, tx;
    if (tiles <= 0x7fffffffLL)
      strip_tile<8, int>(static_cast<int>(t), tiles_x, static_cast<int>(tiles_y), &ty, &tx);
    else
      strip_tile<8, long long>(t, tiles_x, tiles_y, &ty, &tx);
    const int row0 = ty * kVecTile;
    const int col0 = tx * kVecTile;
    if (row0 + kVecTile <= rows && col0 + kVecTile <= cols)
      vec4u_tile<true, kLoadNT, kStoreNT>(input, output, rows, cols, row0, col0, tile);
    else
      vec4u_tile<false, kLoadNT, kStoreNT>(input, output, rows, cols, row0, col0, tile);
    if (t + gridDim.x < tiles) __syncthreads();  // tile is rewritten next
  }
}

// Window transpose, for output rows that are not 16-byte aligned (rows % 4
// != 0 or an unaligned output): every store writes whole, aligned 16-byte
// chunks, and each output row segment a tile writes starts on a 64-byte
// boundary, so no 64-byte block is written partly by two tiles except
// where an output row itself begins or ends inside one.
//   * A tile is kWinCols output rows (input columns col0 ..) by kWinRows
//     output columns (input rows row0 ..). Output row c takes output
//     columns [row0 - d, row0 + kWinRows - d), d = (flat index of (c,
//     row0)) mod 16 -- so the windows of consecutive tiles partition the
//     row, each starting on a 64-byte boundary -- and the last row block
//     runs to `rows` (up to kWinHalo more columns).
//   * The tile therefore needs input rows row0 - 15 .. row0 + kWinRows - 1
//     (a 15-row halo, read again by the tile above). Each input row r is
//     loaded as aligned float4s from column col0 - a(r), a(r) = (flat
//     index of (r, col0)) mod 4: kWinCols / 4 + 1 of them.
// Measured on MI355X against transpose_vec4u_kernel (us; inputs cycling
// through 1 GiB; windows on 128-byte lines, a 31-row halo): 4095x4097 35.2
// -> 29.7, 4097x4095 32.0 -> 27.7, 8191x8193 134.3 -> 105.8, 4095x4096
// 29.3 -> 29.2, 1000x1000 5.5 -> 4.6. Window alignment (us, 4095x4097 /
// 8191x8193): 16 bytes 35.0 / 127.8, 32 bytes 30.7 / 111.4, 64 bytes
// 28.6 / 100.1, 128 bytes 29.7 / 106.0. So partly written 64-byte blocks,
// not the unaligned float4s, cost the time. Where the output rows are
// aligned and only the input rows are not (4096x4095),
// transpose_vec4u_kernel stays faster (28.0 vs 32.4 with 128-byte windows)
// and is kept. Tiles of 128 output rows (85 KiB of LDS, one workgroup per
// CU) took 31.3, 256-column tiles 31.7 (128-byte windows).
constexpr int kWinAlign = 16;                          // floats per 64 bytes
constexpr int kWinHalo = kWinAlign - 1;
constexpr int kWinCols = 64;                           // output rows per tile
constexpr int kWinRows = 128;                          // output columns per tile
constexpr int kWinThreads = 1024;
constexpr int kWinLdsRows = kWinRows + kWinHalo;       // 143 input rows
constexpr int kWinChunks = kWinCols / 4 + 1;           // 17 float4 per input row
constexpr int kWinPitch = 4 * kWinChunks + 1;          // 69 floats
constexpr int kWinLoads = (kWinLdsRows * kWinChunks + kWinThreads - 1) / kWinThreads;  // 3
constexpr int kWinStores = kWinCols * (kWinRows / 4) / kWinThreads;                    // 2
constexpr int kWinExtra = kWinAlign / 4;  // chunks past kWinRows, last row block
static_assert(kWinCols * (kWinRows / 4) % kWinThreads == 0, "whole store passes");

template <bool kFull>
__device__ __forceinline__ void window_tile(const float* __restrict__ input,
                                            float* __restrict__ output, int rows,
                                            int cols, long long total, int row0,
                                            int col0, bool last_r, int off_in,
                                            int off_out, float* lds) {
  const int cols4 = cols & 3;
  const int rowsA = rows & (kWinAlign - 1);
  // LDS row i = input row row0 - kWinHalo + i from column col0 - a(r).
  float4v v[kWinLoads];
#pragma unroll
  for (int n = 0; n < kWinLoads; ++n) {
    const int q = static_cast<int>(threadIdx.x) + kWinThreads * n;
    const int i = q / kWinChunks;
    const int k = q - i * kWinChunks;
    const int r = row0 - kWinHalo + i;
    if (q < kWinLdsRows * kWinChunks && (kFull || (r >= 0 && r < rows))) {
      const int a = ((r & 3) * cols4 + off_in) & 3;
      const long long f = static_cast<long long>(r) * cols + col0 - a + 4 * k;
      if (kFull || (f >= 0 && f + 4 <= total)) {
        // cached: the halo rows are read again by the tile below
        v[n] = *reinterpret_cast<const float4v*>(input + f);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[n][j] = f + j >= 0 && f + j < total ? input[f + j] : 0.0f;
      }
    }
  }
#pragma unroll
  for (int n = 0; n < kWinLoads; ++n) {
    const int q = static_cast<int>(threadIdx.x) + kWinThreads * n;
    if (q < kWinLdsRows * kWinChunks) {
      const int i = q / kWinChunks;
      float* d = lds + i * kWinPitch + 4 * (q - i * kWinChunks);
      d[0] = v[n][0];
      d[1] = v[n][1];
      d[2] = v[n][2];
      d[3] = v[n][3];
    }
  }
  __syncthreads();
  // Chunk k of output row col0 + o: output columns rs .. rs + 3.
  auto store_chunk = [&](int o, int k, bool extra) {
    const int c = col0 + o;
    if (!kFull && c >= cols) return;
    const int d = ((c & (kWinAlign - 1)) * rowsA + off_out) & (kWinAlign - 1);
    const int rs = row0 - d + 4 * k;
    float4v w;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int a = (((j - d) & 3) * cols4 + off_in) & 3;  // a(rs + j)
      // extra chunks store only rows below row0 + kWinRows (LDS rows that exist)
      const int i = extra ? min(kWinHalo - d + 4 * k + j, kWinLdsRows - 1)
                          : kWinHalo - d + 4 * k + j;
      w[j] = lds[i * kWinPitch + o + a];
    }
    float* dst = output + static_cast<long long>(c) * rows + rs;
    if (!extra && (kFull || (rs >= 0 && rs + 4 <= rows))) {
      __builtin_nontemporal_store(w, reinterpret_cast<float4v*>(dst));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (rs + j >= 0 && rs + j < rows) dst[j] = w[j];
    }
  };
#pragma unroll
  for (int n = 0; n < kWinStores; ++n) {
    const int q = static_cast<int>(threadIdx.x) + kWinThreads * n;
    store_chunk(q / (kWinRows / 4), q % (kWinRows / 4), false);
  }
  if (!kFull && last_r) {
    for (int q = static_cast<int>(threadIdx.x); q < kWinCols * kWinExtra; q += kWinThreads)
      store_chunk(q / kWinExtra, kWinRows / 4 + q % kWinExtra, true);
  }
}

// off_in / off_out: the buffers' offsets, in floats, past a 16-byte /
// 64-byte boundary.
__global__ __launch_bounds__(kWinThreads) void transpose_window_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows,
    int cols, int tiles_x, long long tiles, int off_in, int off_out) {
  __shared__ float lds[kWinLdsRows * kWinPitch];
  const long long total = static_cast<long long>(rows) * cols;
  const int tiles_y = static_cast<int>(tiles / tiles_x);
  for (long long t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int ty = static_cast<int>(t / tiles_x);
    const int tx = static_cast<int>(t % tiles_x);
    const int row0 = ty * kWinRows;
    const int col0 = tx * kWinCols;
    const bool last_r = ty == tiles_y - 1;
    // interior: the halo exists, not the last row block, a full column
    // block, every float4 load inside the matrix
    const bool full = row0 >= kWinHalo && !last_r && col0 + kWinCols <= cols &&
                      static_cast<long long>(row0 + kWinRows - 1) * cols + col0 +
                              4 * kWinChunks <= total;
    if (full)
      window_tile<true>(input, output, rows, cols, total, row0, col0, last_r, off_in,
                        off_out, lds);
    else
      window_tile<false>(input, output, rows, cols, total, row0, col0, last_r, off_in,
                         off_out, lds);
    if (t + gridDim.x < tiles) __syncthreads();  // lds is rewritten next
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
  if (rows <= kThinMax || cols <= kThinMax) {
    const int s = rows <= cols ? rows : cols;  // <= kThinMax
    const long long n = rows <= cols ? cols : rows;
    if (n % 4 == 0 && opl::aligned16(input) && opl::aligned16(output)) {
      if (rows <= cols)
        launch_thin4<true>(input, output, s, n, stream);
      else
        launch_thin4<false>(input, output, s, n, stream);
      return hipGetLastError();
    }
    if (rows <= cols)
      launch_thin<true>(input, output, rows, cols, stream);
    else
      launch_thin<false>(input, output, rows, cols, stream);
    return hipGetLastError();
  }
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
  const std::uintptr_t in_addr = reinterpret_cast<std::uintptr_t>(input);
  const std::uintptr_t out_addr = reinterpret_cast<std::uintptr_t>(output);
  // (the window kernel's row and column indices run up to kWinRows /
  // kWinCols past the matrix in 32-bit arithmetic)
  constexpr int kIndexRoom = 0x7fffffff - 2 * kWinRows;
  if (vtiles >= kUnalignedMinTiles && ((in_addr | out_addr) & 3) == 0 &&
      rows < kIndexRoom && cols < kIndexRoom) {
    // Output rows are 16-byte aligned when rows % 4 == 0 and the output is;
    // input rows likewise with cols. This path has at least one side
    // misaligned.
    const bool out_aligned = rows % 4 == 0 && opl::aligned16(output);
    if (out_aligned) {  // only the input rows are misaligned
      const int blocks = static_cast<int>(vtiles < kMaxGrid ? vtiles : kMaxGrid);
      transpose_vec4u_kernel<false, true><<<dim3(blocks), dim3(kThreads), 0, stream>>>(
          input, output, rows, cols, vtiles_x, vtiles);
    } else {
      const int wtiles_x = (cols + kWinCols - 1) / kWinCols;
      const long long wtiles =
          static_cast<long long>(wtiles_x) * ((rows + kWinRows - 1) / kWinRows);
      const int blocks = static_cast<int>(wtiles < kMaxGrid ? wtiles : kMaxGrid);
      transpose_window_kernel<<<dim3(blocks), dim3(kWinThreads), 0, stream>>>(
          input, output, rows, cols, wtiles_x, wtiles, static_cast<int>((in_addr >> 2) & 3),
          static_cast<int>((out_addr >> 2) & (kWinAlign - 1)));
    }
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
