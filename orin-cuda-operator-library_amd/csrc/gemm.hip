// Row-major GEMM C[M,N] = A[M,K] * B[K,N] on the CDNA4 matrix cores.
//   gemm_f16: fp16 A/B, v_mfma_f32_16x16x32_f16 (direct-to-LDS kernel) or
//             v_mfma_f32_32x32x16_f16 (register-staged), fp32 accumulate and output
//   gemm_f32: fp32 A/B, v_mfma_f32_16x16x4_f32 (direct-to-LDS kernel) or
//             v_mfma_f32_32x32x2_f32 (register-staged), fp32 accumulate and output
//
// Reference: operatorlib::gemm_f16 / gemm_f32 (src/gemm.cu:440-479). The
// reference dispatches between WMMA, cp.async register-tiled and scalar
// kernels on divisibility; here the dispatch is, in order:
//   * M <= 16 (decode shapes; the matrix-core one up to 32 fp16 / 64 fp32
//     rows): the skinny kernels (namespace skinny), an HBM stream over B
//     with split K and an ordered split sum;
//   * N <= 16 (matrix-vector products): namespace narrow, an HBM stream
//     over A, one launch;
//   * gemm_dma_kernel (any K, N and alignment, K below 2^22 fp16 / 2^21
//     fp32 and N below 2^24): direct global->LDS loads that read the
//     operands in place, described before the kernel; 256 x 256 tiles, or
//     128 x 128 when the grid would leave CUs idle. Large fp16 products
//     whose rows are not 4-byte aligned (e.g. 4095^3) first copy those
//     operands into chunk-padded rows in scratch (the GPU's arena or the
//     caller's workspace), see PadPlan;
//   * gemm_mfma_kernel, register-staged (Staging below), for K or N past
//     those limits: 16-byte chunks from 16-byte aligned rows (K, N
//     multiples of the chunk, aligned operands), or 16-byte chunks at
//     4-byte alignment (every fp32 shape; fp16 with even K and N), or
//     element-wise with zero fill (any shape and alignment); fp32 uses
//     128 x 128 tiles on small grids.
// Every path but the vector-ALU skinny kernel (M <= 4 fp16, M <= 8 fp32)
// runs on the matrix cores.
//
// Register-staged tiling (gemm_mfma_kernel, both precisions):
//   * 256 x 256 C tile per workgroup. fp16: 2 x 2 wavefronts (256 threads),
//     each owning a 128 x 128 sub-tile = 4 x 4 MFMA 32x32 blocks (256 fp32
//     accumulators per lane, one wave per SIMD). fp32: 2 x 4 wavefronts
//     (512 threads) of 128 x 64, two waves per SIMD (WaveLayout below);
//   * K step of 128 bytes per row (64 fp16 or 32 fp32): both operands are
//     kept "k-contiguous" in LDS (A as [m][k], B transposed to [n][k]) so
//     every MFMA operand is one ds_read_b128;
//   * B is transposed in registers while it is staged (8x8 fp16 or 4x4
//     fp32 blocks), because row-major B is n-contiguous;
//   * LDS rows are padded to 144 bytes, which spreads both the 16-row
//     operand reads and the staging writes over the LDS banks;
//   * two LDS stages: global loads for step k+1 are in flight while step k
//     runs on the matrix cores; one barrier per K step;
//   * workgroups are renumbered so that each XCD (blocks are dealt to the
//     8 XCDs round-robin) works on a compact group of tiles, for L2 reuse.
//
// MFMA operand lanes: lane l supplies row/column (l % 32) and the k-chunk
// selected by (l / 32). Any assignment of k values to (lane half, element)
// gives the same product as long as A and B use the same one, and both are
// read with the identical pattern below. The 32x32 accumulator layout is
// the CDNA one: element i of lane l is C[8*(i/4) + 4*(l/32) + i%4][l % 32].

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "scratch.hpp"
#include "validate.hpp"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kRowBytes = 128;        // one K step of one row
constexpr int kChunksPerRow = kRowBytes / 16;
constexpr int kPitch = kRowBytes + 16;  // padded LDS row
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

template <typename T>
struct Precision;

template <>
struct Precision<_Float16> {
  using Chunk = half8;
  static constexpr int kChunkElems = 8;
  __device__ __forceinline__ static void mma(floatx16& acc, const Chunk& a,
                                             const Chunk& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
};

template <>
struct Precision<float> {
  using Chunk = float4v;
  static constexpr int kChunkElems = 4;
  __device__ __forceinline__ static void mma(floatx16& acc, const Chunk& a,
                                             const Chunk& b) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);
  }
};

// Tile and wavefront layout of the register-staged kernel: a BM x BN C tile
// per workgroup, WM x WN wavefronts, WavesPerSimd wavefronts resident per
// SIMD (the register budget follows from it).
//   * fp16: 256 x 256, 2 x 2 wavefronts of 128 x 128, one per SIMD;
//   * fp32: 256 x 256, 2 x 4 wavefronts of 128 x 64, two per SIMD, whose
//     second wavefront covers the first one's staging and barrier waits
//     (4096^3: 133.1 -> 135.5 TFLOP/s, results bit-identical);
//   * fp32 on grids that 256 x 256 tiles would leave mostly idle:
//     128 x 128, 2 x 2 wavefronts of 64 x 64, two workgroups per CU.
template <int WM, int WN, int BM, int BN, int WavesPerSimd>
struct WaveLayout {
  static constexpr int kWM = WM;
  static constexpr int kWN = WN;
  static constexpr int kBM = BM;
  static constexpr int kBN = BN;
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int kWaveM = BM / WM;
  static constexpr int kWaveN = BN / WN;
  static constexpr int kFragsM = kWaveM / 32;
  static constexpr int kFragsN = kWaveN / 32;
  static constexpr int kWavesPerSimd = WavesPerSimd;
  static constexpr int kTileABytes = BM * kPitch;
  static constexpr int kTileBBytes = BN * kPitch;
  static constexpr int kStageBytes = kTileABytes + kTileBBytes;
  static constexpr int kLdsBytes = 2 * kStageBytes;
};

using F16Layout = WaveLayout<2, 2, 256, 256, 1>;
using F32Layout = WaveLayout<2, 4, 256, 256, 2>;
using F32SmallLayout = WaveLayout<2, 2, 128, 128, 2>;

template <typename T>
struct LayoutFor {
  using type = F16Layout;
};
template <>
struct LayoutFor<float> {
  using type = F32Layout;
};

// How gemm_mfma_kernel stages its operands from global memory:
//   * kElementwise: element by element with zero fill (any shape and
//     alignment);
//   * kAligned16: one 16-byte load per chunk; rows are 16-byte aligned
//     (K, N multiples of the chunk, 16-byte aligned A and B), so a chunk is
//     wholly inside or outside a row;
//   * kDword: one 16-byte load per chunk at 4-byte alignment (every fp32
//     matrix; fp16 ones with even K and N and 4-byte aligned A and B); a
//     chunk that runs past its row's end is loaded element by element, so
//     no load reaches past a row (or the matrix).
enum Staging { kElementwise, kAligned16, kDword };

template <typename T, int kStaging, typename L>
struct Stager {
  using P = Precision<T>;
  using Chunk = typename P::Chunk;
  static constexpr int E = P::kChunkElems;
  static constexpr int kBK = kRowBytes / sizeof(T);  // K elements per step
  static constexpr int kThreads = L::kThreads;
  // A: BM rows x kChunksPerRow chunks; each thread stages kAChunks.
  static constexpr int kAChunks = L::kBM * kChunksPerRow / kThreads;
  // B: E x E element blocks (E k-rows x one n-chunk); kBBlocks per thread.
  static constexpr int kBBlocks = (kBK / E) * (L::kBN / E) / kThreads;
  static_assert(kAChunks * kThreads == L::kBM * kChunksPerRow &&
                    kBBlocks >= 1 && kBBlocks * kThreads == (kBK / E) * (L::kBN / E),
                "staging work must divide evenly over the workgroup");

  Chunk a[kAChunks];
  Chunk b[kBBlocks][E];

  __device__ __forceinline__ static Chunk load_chunk(const T* base,
                                                     std::size_t ld, int row,
                                                     int rows, int col,
                                                     int cols) {
    Chunk v;
    if constexpr (kStaging == kAligned16) {
      // cols % E == 0, so a chunk is all in or out.
      if (row < rows && col < cols) {
        v = *reinterpret_cast<const Chunk*>(
            base + static_cast<std::size_t>(row) * ld + col);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = T(0);
      }
    } else if constexpr (kStaging == kDword) {
      typedef Chunk DwordChunk __attribute__((aligned(4)));
      const T* p = base + static_cast<std::size_t>(row) * ld;
      if (row < rows && col + E <= cols) {
        v = *reinterpret_cast<const DwordChunk*>(p + col);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
          v[e] = (row < rows && col + e < cols) ? p[col + e] : T(0);
      }
    } else {
      const T* p = base + static_cast<std::size_t>(row) * ld;
#pragma unroll
      for (int e = 0; e < E; ++e)
        v[e] = (row < rows && col + e < cols) ? p[col + e] : T(0);
    }
    return v;
  }

  // Global -> registers for the K step starting at k0.
  __device__ __forceinline__ void load(const T* A, const T* B, int M, int ldb,
                                       int K, int m0, int n0, int k0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAChunks; ++i) {
      const int q = tid + kThreads * i;
      const int row = q / kChunksPerRow;
      const int c = q % kChunksPerRow;
      a[i] = load_chunk(A, K, m0 + row, M, k0 + c * E, K);
    }
#pragma unroll
    for (int blk = 0; blk < kBBlocks; ++blk) {
      const int q = tid + kThreads * blk;
      const int g = q % (kBK / E);  // k-chunk within the step
      const int j = q / (kBK / E);  // n-chunk
#pragma unroll
      for (int r = 0; r < E; ++r)
        b[blk][r] = load_chunk(B, ldb, k0 + g * E + r, K, n0 + j * E, ldb);
    }
  }

  // Registers -> LDS stage (A as [m][k], B transposed to [n][k]).
  __device__ __forceinline__ void store(unsigned char* stage) const {
    const int tid = threadIdx.x;
    unsigned char* sa = stage;
    unsigned char* sb = stage + L::kTileABytes;
#pragma unroll
    for (int i = 0; i < kAChunks; ++i) {
      const int q = tid + kThreads * i;
      const int row = q / kChunksPerRow;
      const int c = q % kChunksPerRow;
      *reinterpret_cast<Chunk*>(sa + row * kPitch + c * 16) = a[i];
    }
#pragma unroll
    for (int blk = 0; blk < kBBlocks; ++blk) {
      const int q = tid + kThreads * blk;
      const int g = q % (kBK / E);
      const int j = q / (kBK / E);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        Chunk t;
#pragma unroll
        for (int r = 0; r < E; ++r) t[r] = b[blk][r][i];
        *reinterpret_cast<Chunk*>(sb + (j * E + i) * kPitch + g * 16) = t;
      }
    }
  }
};

// Tile `idx` of the grouped order: column-major groups of kGroupM tile-rows.
__device__ __forceinline__ void grouped_tile(int idx, int tiles_m, int tiles_n,
                                             int* tm, int* tn) {
  const int group_size = kGroupM * tiles_n;
  const int first_m = (idx / group_size) * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int in_group = idx % group_size;
  *tm = first_m + in_group % rows_in_group;
  *tn = in_group / rows_in_group;
}

// Launch index b of `blocks` -> grouped-order index: regroups the
// round-robin XCD dispatch so that consecutive tiles land on one XCD.
__device__ __forceinline__ int xcd_regroup(int b, int blocks) {
  return blocks % kXcds == 0 ? (b % kXcds) * (blocks / kXcds) + b / kXcds : b;
}

// Maps the launch index to a C tile: XCD regrouping, then the grouped order.
__device__ __forceinline__ void tile_of_block(int tiles_m, int tiles_n,
                                              int* tm, int* tn) {
  grouped_tile(xcd_regroup(blockIdx.x, gridDim.x), tiles_m, tiles_n, tm, tn);
}

// Grids of whole 16 x 16 blocks of tiles with one workgroup per CU: each
// round of 256 workgroups (one per CU) takes one 16 x 16 super-tile, and XCD
// x an 8 x 4 block of it, in column-major order within the block. A round
// then reads 16 tile rows of A and 16 tile columns of B, where the grouped
// order above spreads a round over all tile rows (8192 x 8192 tiles of 256:
// 32 tile rows and 8 tile columns). Measured on MI355X, fp16, us (grouped
// vs super-tiles): 8192 x 8192 x 4096 500 vs 458, 16384 x 4096 x 4096 486
// vs 475, 8192^3 910 vs 909, 4096^3 117 vs 117 (the same order there).
// Needs gridDim.x = tiles_m * tiles_n with tiles_m, tiles_n % 16 == 0.
__device__ __forceinline__ void super_tile_of_block(int tiles_n, int* tm, int* tn) {
  const int x = blockIdx.x % kXcds;   // XCD (workgroups are dealt round-robin)
  const int j = blockIdx.x / kXcds;   // this XCD's j-th workgroup
  const int round = j / 32;           // 32 workgroups per XCD and round
  const int q = j % 32;
  const int super_cols = tiles_n / 16;
  *tm = (round / super_cols) * 16 + (x / 4) * 8 + q % 8;
  *tn = (round % super_cols) * 16 + (x % 4) * 4 + q / 8;
}

template <typename T, int kStaging, typename L = typename LayoutFor<T>::type>
__global__ __launch_bounds__(L::kThreads)
__attribute__((amdgpu_waves_per_eu(L::kWavesPerSimd, L::kWavesPerSimd)))
void gemm_mfma_kernel(const T* __restrict__ A, const T* __restrict__ B,
                      float* __restrict__ C, int M, int N, int K, int ldb) {
  using P = Precision<T>;
  using Chunk = typename P::Chunk;
  using S = Stager<T, kStaging, L>;
  constexpr int kBM = L::kBM;
  constexpr int kBN = L::kBN;
  constexpr int kTileABytes = L::kTileABytes;
  constexpr int kStageBytes = L::kStageBytes;
  constexpr int kWaveM = L::kWaveM;
  constexpr int kWaveN = L::kWaveN;
  constexpr int kFragsM = L::kFragsM;
  constexpr int kFragsN = L::kFragsN;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::kLdsBytes];

  const int tiles_m = (M + kBM - 1) / kBM;
  const int tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of_block(tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;

  const int lane = threadIdx.x % opl::kWaveSize;
  const int wave = threadIdx.x / opl::kWaveSize;
  const int wm = wave / L::kWN;
  const int wn = wave % L::kWN;
  const int half = lane / 32;
  const int l32 = lane % 32;

  floatx16 acc[kFragsM][kFragsN];
#pragma unroll
  for (int i = 0; i < kFragsM; ++i)
#pragma unroll
    for (int j = 0; j < kFragsN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  const int steps = (K + S::kBK - 1) / S::kBK;
  S stager;
  stager.load(A, B, M, ldb, K, m0, n0, 0);
  stager.store(lds);
  __syncthreads();

  // Byte offsets of this lane's operand rows inside a stage.
  int a_row[kFragsM], b_row[kFragsN];
#pragma unroll
  for (int i = 0; i < kFragsM; ++i)
    a_row[i] = (wm * kWaveM + 32 * i + l32) * kPitch;
#pragma unroll
  for (int j = 0; j < kFragsN; ++j)
    b_row[j] = kTileABytes + (wn * kWaveN + 32 * j + l32) * kPitch;

  for (int step = 0; step < steps; ++step) {
    const unsigned char* stage = lds + (step & 1) * kStageBytes;
    if (step + 1 < steps)
      stager.load(A, B, M, ldb, K, m0, n0, (step + 1) * S::kBK);
#pragma unroll
    for (int p = 0; p < kChunksPerRow / 2; ++p) {
      const int chunk = (2 * p + half) * 16;
      Chunk a[kFragsM], b[kFragsN];
#pragma unroll
      for (int i = 0; i < kFragsM; ++i)
        a[i] = *reinterpret_cast<const Chunk*>(stage + a_row[i] + chunk);
#pragma unroll
      for (int j = 0; j < kFragsN; ++j)
        b[j] = *reinterpret_cast<const Chunk*>(stage + b_row[j] + chunk);
#pragma unroll
      for (int i = 0; i < kFragsM; ++i)
#pragma unroll
        for (int j = 0; j < kFragsN; ++j) P::mma(acc[i][j], a[i], b[j]);
    }
    if (step + 1 < steps) stager.store(lds + ((step + 1) & 1) * kStageBytes);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < kFragsM; ++i) {
#pragma unroll
    for (int j = 0; j < kFragsN; ++j) {
      const int col = n0 + wn * kWaveN + 32 * j + l32;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row =
            m0 + wm * kWaveM + 32 * i + 8 * (e / 4) + 4 * half + (e % 4);
        if (row < M && col < N)
          C[static_cast<std::size_t>(row) * N + col] = acc[i][j][e];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// gemm_dma_kernel — the fast path of both precisions (16-byte aligned A
// and B; fp16: K % 32 == 0, N % 8 == 0; fp32: K % 16 == 0, N % 4 == 0).
// Described for fp16; fp32 differences at the end.
//
//   * 256 x 256 C tile per 512-thread workgroup: 8 wavefronts as 2 (M) x 4
//     (N), each owning 128 x 64 = 8 x 4 MFMA 16x16x32 blocks (128 fp32
//     accumulators, so two wavefronts fit per SIMD and one's LDS waits are
//     covered by the other's MFMAs);
//   * grids of fewer than 160 such tiles (medium M or N) use 128 x 128
//     tiles instead: 4 wavefronts of 64 x 64, four times the workgroups,
//     about 2x faster where 256 x 256 tiles would leave most CUs idle;
//   * v_mfma_f32_16x16x32_f16 rather than 32x32x16: the same LDS bytes per
//     flop and bit-identical sums, but the GPU holds a higher clock under
//     the power limit with it (MI355X, a loop of MFMAs alone: 1.99 against
//     1.70 GHz; with the GEMM's LDS reads: 1.75 against 1.55 GHz);
//   * A and B are copied global -> LDS by buffer loads with the lds
//     modifier (each lane writes 16 bytes at LDS base + 16 * lane) from
//     per-step scalar bases, so operands never pass through VGPRs and no
//     ds_write is issued;
//   * both tiles keep their global layout (A [m][k], B [k][n]); B fragments
//     are read with ds_read_b64_tr_b16, which returns k-contiguous fp16
//     pairs from n-contiguous rows: within each 16-lane group, lane 4r + j
//     addresses 4 elements of row r and lane i receives element i % 4 of
//     the lanes 4r + i / 4, r = 0..3;
//   * XOR swizzles of the 16-byte chunks make every read conflict-free:
//     A rows of 128 B (64-deep stages) use chunk ^ ((m >> 1) & 7), rows of
//     64 B (32-deep stages) chunk ^ ((m >> 2) & 3); B rows chunk ^ 4 * (k &
//     3) ^ 2 * (bit 3 of k); the DMA lane -> chunk mapping applies the same
//     swizzle, and it keeps contiguous global segments per row;
//   * stages in separate LDS arrays (so the compiler can see that the DMA
//     into one does not alias the reads of another). Every 32-deep substep
//     reads the next substep's fragments under its MFMAs, one LDS read or
//     DMA issue after an MFMA at a time (sched_group_barrier);
//   * 256 x 256 tiles with K % 64 == 0: two 64-deep stages, each step two
//     substeps, the barrier between them: by then every wave has read its
//     last fragments from the stage and the next stage has landed, so the
//     second substep's MFMAs cover both the next step's first fragment
//     reads and the DMA refill of the stage just finished;
//   * 128 x 128 tiles and K % 64 == 32: four 32-deep stages, one substep
//     and one barrier per step, copies issued three steps ahead (partial
//     vmcnt waits). Measured against the two-stage schedule (us): 2048^3
//     22.8 vs 27.6, 1000^3 19.6 vs 23.2 (128 x 128 tiles); 256 x 256 tiles
//     lose (4096^3 109.6 vs 104.2), as their per-step barrier costs more
//     than the deeper prefetch saves;
//   * copies of steps past the end read through an empty buffer range
//     (zeros, no memory access), so every step runs the same code;
//   * M / N edges: source rows past M are clamped to M - 1, columns past N
//     read whatever follows (their results are never stored), stores are
//     masked; a partly filled last K step is repaired in LDS (fix_stage);
//   * any row length and alignment: a 16-byte direct-to-LDS copy from any
//     byte address lands whole, so rows are read in place. Rows at a 2-byte
//     phase (fp16, odd K or N) cost time, dword-aligned ones nothing (us,
//     MI355X: fp32 4095^3 925 against 979 on padded copies; fp16 4096 x
//     4096 x 4095 114 against 128; 1000^3 19 against 32; 100^3 6 against
//     15).
//   * C leaves through LDS as full-line 16-byte stores, non-temporal on
//     grids of two or more rounds with large operands (store_staged and
//     the launcher's stream_c rule).
// Measured on MI355X (median of 8-launch groups): 4096^3 100-105 us, 8192^3
// 740-780 us (1.41-1.49 PFLOP/s); hipBLASLt with the same fp32 C: 114 and
// 853-856 us. Before the staged epilogue: 104-109 / 852-871 us. With
// v_mfma_f32_32x32x16_f16 the same schedule ran 111-119 / 890-910 us,
// bit-identical output.
//
// fp32: the same tiles, stages and schedule with the same A row bytes per
// step (32 or 16 elements), on v_mfma_f32_16x16x4_f32. A fragments are the
// same 16-byte chunks; B rows (1 KiB for 256-wide tiles) are read with one
// ds_read_b32 per lane and MFMA (lane group q reads row 4q + e of the
// substep, e = 0..3, and A's chunk q), and swizzled chunk ^ 4 * ((k >> 2) &
// 3) so the four lane groups of a read hit different banks. A substep is
// 16 deep, 4 MFMAs per 16 x 16 block, interleaved with the reads and copies
// in groups of one block's 4 MFMAs. The fp32 MFMA rate does not fall under
// load (a loop of them alone: 155 TFLOP/s, 0.99 of peak), so what the
// register-staged kernel lost to its VGPR staging, transposes and LDS
// writes comes back. Measured on MI355X (us, register-staged -> direct):
// 4096^3 1017 -> 928 (0.94 of the fp32 peak; hipBLASLt 964-979), 8192 x
// 8192 x 4096 4050 -> 3697, 2048^3 153.5 -> 124.5, 1000 x 4096 x 4096
// 301 -> 242, 4352 x 4096 x 1024 (split last round) 515 -> 326.
// ---------------------------------------------------------------------------

namespace dma {

typedef __fp16 fp16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Split of a grid's last, partly filled round (or of every tile of a grid
// too small to fill the CUs, full_tiles = 0): launch indices below
// full_tiles take whole tiles; the `tiles` tiles after them in the grouped
// order are each cut into `splits` contiguous K ranges, one workgroup per
// range, written to `partial` ([splits][tiles][BM x BN] fp32, rows past M
// left unwritten) and summed by sum_tail_kernel. splits == 0: no split,
// one workgroup per tile.
struct TailSplit {
  int full_tiles;
  int tiles;
  int splits;
  float* partial;
};
#define OPL_LDS __attribute__((address_space(3)))

// Element types of the direct-to-LDS kernel. A substep is the k range one
// set of fragments covers: every operand fragment is 16 bytes per lane.
//   * fp16: one v_mfma_f32_16x16x32_f16 per 16 x 16 block and substep of
//     32; A and B fragments are 8 k-contiguous halves (B read transposed);
//   * fp32: four v_mfma_f32_16x16x4_f32 per block and substep of 16. Lane
//     group q (lanes 16q..16q+15) reads A's 16-byte chunk q of the substep
//     (k = 4q..4q+3) and, for MFMA e, B's row 4q + e: so MFMA e multiplies
//     k = 4q + e in every lane group, on both operands.
template <typename T>
struct Elem;
template <>
struct Elem<_Float16> {
  using Frag = half8;
  static constexpr int kSubK = 32;
  static constexpr int kMfmas = 1;  // MFMAs per 16 x 16 block and substep
  static constexpr int kBReads = 2;  // LDS reads per B fragment
};
template <>
struct Elem<float> {
  using Frag = floatx4;
  static constexpr int kSubK = 16;
  static constexpr int kMfmas = 4;
  static constexpr int kBReads = 4;
};

// C tile configurations. BM x BN per workgroup, WM x WN wavefronts of
// (BM / WM) x (BN / WN); K steps of BK elements (128 or 64 bytes of an A
// row) in `Stages` LDS stages. B rows in LDS are BN elements (BN *
// sizeof(T) / 16 16-byte chunks).
template <typename T, int BM, int BN, int WM, int WN, int BK, int Stages>
struct Tile {
  using Type = T;
  using Frag = typename Elem<T>::Frag;
  static constexpr int kBM = BM, kBN = BN, kBK = BK;
  static constexpr int kWM = WM, kWN = WN;
  static constexpr int kStages = Stages;
  static constexpr int kSubsteps = BK / Elem<T>::kSubK;  // fragment sets per step
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int kFM = BM / WM / 16;
  static constexpr int kFN = BN / WN / 16;
  static constexpr int kChunkElems = 16 / static_cast<int>(sizeof(T));
  static constexpr int kARowBytes = BK * static_cast<int>(sizeof(T));
  static constexpr int kAChunks = kARowBytes / 16;
  static constexpr int kABytes = BM * kARowBytes;
  static constexpr int kBRowBytes = BN * static_cast<int>(sizeof(T));
  static constexpr int kBBytes = BK * kBRowBytes;
  static constexpr int kBChunks = kBRowBytes / 16;
  static constexpr int kStage = kABytes + kBBytes;
  // DMA chunks per thread per operand.
  static constexpr int kCopies = kABytes / 16 / kThreads;
  static_assert(kABytes == kBBytes && kCopies * 16 * kThreads == kABytes,
                "both operand tiles split evenly into 16-byte copies");
  static_assert(64 % kBChunks == 0, "a wavefront copies whole B rows");
  static_assert((kARowBytes == 128 && Stages == 2) || (kARowBytes == 64 && Stages == 4),
                "two 128-byte or four 64-byte stages of A rows");
  // XOR swizzle of A row m's 16-byte chunks: rows 16 apart share it.
  __device__ static int swizzle_a(int m) {
    return kAChunks == 8 ? (m >> 1) & 7 : (m >> 2) & 3;
  }
  // XOR swizzle of B row k's 16-byte chunks. fp16 (ds_read_b64_tr_b16 of
  // rows k & 3 and bit 3 of k): chunk ^ 4 * (k & 3) ^ 2 * (bit 3 of k).
  // fp32 (ds_read_b32, the 16-lane groups of one read on rows 4 apart):
  // chunk ^ 4 * ((k >> 2) & 3), so the four groups' 64-byte row segments
  // fall on four different 64-byte bank ranges.
  __device__ static int swizzle_b(int k) {
    if constexpr (sizeof(T) == 2)
      return 4 * (k & 3) ^ 2 * ((k >> 3) & 1);
    else
      return 4 * ((k >> 2) & 3);
  }
};
// 256 x 256: 8 wavefronts of 128 x 64, for grids that fill the GPU.
using BigTile = Tile<_Float16, 256, 256, 2, 4, 64, 2>;
// The same for K % 64 == 32.
using BigTileK32 = Tile<_Float16, 256, 256, 2, 4, 32, 4>;
// 128 x 128: 4 wavefronts of 64 x 64, four times the workgroups for the
// same C, for grids that would leave CUs idle with BigTile.
using SmallTile = Tile<_Float16, 128, 128, 2, 2, 32, 4>;
// fp32: the same geometry with the same A row bytes per step (32 or 16
// elements).
using BigTileF32 = Tile<float, 256, 256, 2, 4, 32, 2>;
using BigTileF32K16 = Tile<float, 256, 256, 2, 4, 16, 4>;
using SmallTileF32 = Tile<float, 128, 128, 2, 2, 16, 4>;

template <typename Cfg>
struct Fragments {
  typename Cfg::Frag a[Cfg::kFM];
  typename Cfg::Frag b[Cfg::kFN];
};

template <typename Cfg, bool kTail = false, bool kEdge = false, bool kStreamC = false>
__global__ __launch_bounds__(Cfg::kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_dma_kernel(const typename Cfg::Type* __restrict__ A,
                     const typename Cfg::Type* __restrict__ B,
                     float* __restrict__ C, int M, int N, int K, int lda, int ldb,
                     TailSplit tail) {
  using T = typename Cfg::Type;
  using E = Elem<T>;
  constexpr int kBM = Cfg::kBM, kBN = Cfg::kBN, kBK = Cfg::kBK;
  constexpr int kWM = Cfg::kWM, kWN = Cfg::kWN;
  constexpr int kFM = Cfg::kFM, kFN = Cfg::kFN;
  constexpr int kABytes = Cfg::kABytes, kCopies = Cfg::kCopies;
  constexpr int kBChunks = Cfg::kBChunks;
  constexpr int kSize = static_cast<int>(sizeof(T));
  constexpr int kReads = kFM + E::kBReads * kFN;  // LDS read instructions per substep
  constexpr int kIssues = 2 * kCopies;            // DMA instructions per K step
  static_assert(kWM == 2, "A fragment offsets assume two wavefront rows");

  const int tiles_m = (M + kBM - 1) / kBM;
  const int tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  // K steps [kstep0, kstep0 + steps) of the tile; split >= 0: a tail part
  // (kTail instances only; the others keep kstep0 = 0 at compile time).
  int kstep0 = 0;
  const int total_steps = (K + kBK - 1) / kBK;
  int steps = total_steps;
  int split = -1, tail_index = 0;
  if constexpr (kTail) {
    const int b = blockIdx.x;
    if (b < tail.full_tiles) {
      grouped_tile(xcd_regroup(b, tail.full_tiles), tiles_m, tiles_n, &tm, &tn);
    } else {
      const int w = b - tail.full_tiles;
      tail_index = w / tail.splits;
      split = w % tail.splits;
      grouped_tile(tail.full_tiles + tail_index, tiles_m, tiles_n, &tm, &tn);
      const int per = steps / tail.splits, extra = steps % tail.splits;
      kstep0 = split * per + min(split, extra);
      steps = per + (split < extra ? 1 : 0);
    }
  } else if (kBM == 256 && tiles_m % 16 == 0 && tiles_n % 16 == 0) {
    // 256 x 256 tiles run one workgroup per CU (128 KiB of LDS)
    super_tile_of_block(tiles_n, &tm, &tn);
  } else {
    tile_of_block(tiles_m, tiles_n, &tm, &tn);
  }
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;

  const int lane = threadIdx.x % opl::kWaveSize;
  // wave-uniform, so each copy's LDS destination is a scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / opl::kWaveSize);
  const int wm = wave / kWN;
  const int wn = wave % kWN;
  const int group = lane / 16;
  const int gl = lane % 16;

  // DMA sources: copy j of this thread fills LDS chunk slot
  // (wave * kCopies + j) * 64 + lane of each operand tile. They are byte
  // offsets from the step's scalar bases A + m0 * lda + k0 and
  // B + k0 * ldb + n0 (A rows clamped to M - 1), read through buffer
  // resources: no 64-bit vector address math per copy. The copies need no
  // alignment: a 16-byte copy from any byte address lands whole (measured
  // on MI355X at every byte phase, at the aligned copy rate), so rows of
  // any length are read in place. A chunk that runs past its row's end
  // reads the next row's first elements: past N those fill columns that
  // are never stored; past K, see fix_stage.
  int a_dma[kCopies];
  int b_dma[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; ++j) {
    const int slot = (wave * kCopies + j) * 64 + lane;
    const int m = slot / Cfg::kAChunks;
    const int chunk = (slot % Cfg::kAChunks) ^ Cfg::swizzle_a(m);
    a_dma[j] = (min(m0 + m, M - 1) - m0) * lda * kSize + 16 * chunk;
    const int kk = (wave * kCopies + j) * (64 / kBChunks) + lane / kBChunks;
    const int col = Cfg::kChunkElems * ((lane % kBChunks) ^ Cfg::swizzle_b(kk));
    b_dma[j] = kk * ldb * kSize + col * kSize;
  }
  // Bytes from a step's base to the end of its operand, capped at the
  // 32-bit range (every offset above stays far below it). Steps past the
  // end get an empty range: their copies read zeros and touch no memory.
  auto span = [](long long bytes) {
    return static_cast<unsigned>(bytes < 0xffffffffLL ? bytes : 0xffffffffLL);
  };
  // Operand origins of this tile's first K step (kstep0 > 0: a tail part).
  const T* const a_tile = A + static_cast<std::size_t>(m0) * lda + kstep0 * kBK;
  const T* const b_tile = B + static_cast<std::size_t>(kstep0) * kBK * ldb + n0;
  const long long a_total =
      static_cast<long long>(M - m0) * lda * kSize - static_cast<long long>(kSize) * kstep0 * kBK;
  const long long b_total =
      (static_cast<long long>(K) - static_cast<long long>(kstep0) * kBK) * ldb * kSize -
      static_cast<long long>(kSize) * n0;
  // A last K step that is only partly inside the matrix (K % kBK != 0):
  // its copies run each A row past column K into the next row's first
  // elements (B's rows past K lie past B's end and read zeros). The range
  // check zeroes whole dwords, so with fp16 the dword that holds the last
  // element of A (odd lda) or of B (odd ldb) together with the first bytes
  // past the end reads as zero as well. That step runs first (local step 0
  // copies global step kstep0 + steps - 1, the others follow in order), so
  // fix_stage repairs it in LDS once, before the K loop: A's columns past K
  // become zeros and the two end elements are written from copies loaded
  // at the start. One barrier per tile; the loop itself stays as it is (a
  // repair inside it cost the fp16 kernel 24 VGPRs and spills).
  const int k_last = K - (total_steps - 1) * kBK;  // valid k of the last step
  const bool a_past_k = k_last < kBK;
  const bool a_end = kSize == 2 && (lda & 1) != 0 && m0 + kBM >= M;
  const bool b_end = kSize == 2 && (ldb & 1) != 0 && n0 + kBN >= ldb;
  const bool fix = kEdge && kstep0 + steps == total_steps && (a_past_k || b_end);

  auto issue = [&](unsigned char* stage, int kstep) {
    const unsigned live = kstep < steps ? ~0u : 0u;
    const int k0 = (fix ? (kstep == 0 ? steps - 1 : kstep - 1) : kstep) * kBK;
    const unsigned a_span = span(a_total - static_cast<long long>(kSize) * k0) & live;
    const unsigned b_span = span(b_total - static_cast<long long>(kSize) * k0 * ldb) & live;
    const T* a_base = a_tile + k0;
    const T* b_base = b_tile + static_cast<std::size_t>(k0) * ldb;
#pragma unroll
    for (int j = 0; j < kCopies; ++j) {
      opl::buffer_copy16_lds(a_base, a_span, stage + (wave * kCopies + j) * 1024,
                             a_dma[j]);
      opl::buffer_copy16_lds(b_base, b_span, stage + kABytes + (wave * kCopies + j) * 1024,
                             b_dma[j]);
    }
  };

  __shared__ T end_elems[2];
  T a_end_value = T(0), b_end_value = T(0);
  if (fix && threadIdx.x == 0) {
    if (a_end) a_end_value = A[static_cast<std::size_t>(M) * lda - 1];
    if (b_end) b_end_value = B[static_cast<std::size_t>(K) * ldb - 1];
  }
  // Called on stage 0 after the first barrier.
  auto fix_stage = [&](unsigned char* st) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    constexpr int E = Cfg::kChunkElems;
    OPL_LDS unsigned char* const s = (OPL_LDS unsigned char*)st;
    const int tid = threadIdx.x;
    if (a_past_k) {
      for (int m = tid; m < kBM; m += Cfg::kThreads) {
        OPL_LDS unsigned char* const row = s + m * Cfg::kARowBytes;
        const int sw = Cfg::swizzle_a(m);
        if (k_last % E != 0) {  // the chunk across column K, element by element
          OPL_LDS T* const c = (OPL_LDS T*)(row + (((k_last / E) ^ sw) * 16));
          for (int e = k_last % E; e < E; ++e) c[e] = T(0);
        }
        for (int c = (k_last + E - 1) / E; c < Cfg::kAChunks; ++c)
          *(OPL_LDS u32x4*)(row + ((c ^ sw) * 16)) = u32x4{0u, 0u, 0u, 0u};
      }
      if (a_end && tid == 0) {
        const int m = M - 1 - m0, kk = k_last - 1;
        ((OPL_LDS T*)(s + m * Cfg::kARowBytes + (((kk / E) ^ Cfg::swizzle_a(m)) * 16)))[kk % E] =
            end_elems[0];
      }
    }
    if (b_end && tid == 0) {
      const int kk = k_last - 1, n = ldb - 1 - n0;
      ((OPL_LDS T*)(s + kABytes + kk * Cfg::kBRowBytes +
                    (((n / E) ^ Cfg::swizzle_b(kk)) * 16)))[n % E] = end_elems[1];
    }
    // s_waitcnt lgkmcnt(0), copies left in flight; then every wave's writes
    // are in place
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("s_barrier" ::: "memory");
  };

  // Fragment byte offsets inside a stage (lane l supplies row / column
  // l % 16 of its operands and the 16-byte k chunk l / 16 of a substep).
  // A: row m = wm * BM / 2 + 16 ti + l % 16 has the same swizzle for every
  // ti (rows 16 apart), so one VGPR per substep s serves every ti. B, fp16:
  // k & 3 and bit 3 of k are the same for every s and both 4-row halves;
  // fp32: rows 16 s + 4 group + e share the swizzle of row 4 group. Either
  // way one VGPR per tj serves every s (and half, or e).
  constexpr int kBSubstep = E::kSubK * Cfg::kBRowBytes;
  unsigned a_lane[Cfg::kSubsteps];
  {
    const int m = wm * (kBM / kWM) + gl;
#pragma unroll
    for (int s = 0; s < Cfg::kSubsteps; ++s)
      a_lane[s] = m * Cfg::kARowBytes + (((4 * s + group) ^ Cfg::swizzle_a(m)) * 16);
  }
  unsigned b_lane[kFN];
#pragma unroll
  for (int tj = 0; tj < kFN; ++tj) {
    if constexpr (kSize == 2) {
      const int n = wn * (kBN / kWN) + 16 * tj + 4 * (gl % 4);
      const int k = 8 * group + gl / 4;
      b_lane[tj] = kABytes + k * Cfg::kBRowBytes + (((n / 8) ^ Cfg::swizzle_b(k)) * 16) +
                   (n % 8) * 2;
    } else {
      const int n = wn * (kBN / kWN) + 16 * tj + gl;
      const int k = 4 * group;
      b_lane[tj] = kABytes + k * Cfg::kBRowBytes + (((n / 4) ^ Cfg::swizzle_b(k)) * 16) +
                   (n % 4) * 4;
    }
  }

  floatx4 acc[kFM][kFN];
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;

  // Fragments of substep s, read in the order the MFMAs use them (ti-major):
  // A 0, every B, then the other A.
  auto load_a = [&](const unsigned char* st, int s, Fragments<Cfg>& f, int t) {
    f.a[t] = *reinterpret_cast<const typename Cfg::Frag*>(st + a_lane[s] +
                                                          t * 16 * Cfg::kARowBytes);
  };
  auto load = [&](const unsigned char* st, int s, Fragments<Cfg>& f) {
    load_a(st, s, f, 0);
#pragma unroll
    for (int t = 0; t < kFN; ++t) {
      if constexpr (kSize == 2) {
        const fp16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            (OPL_LDS fp16x4*)(st + b_lane[t] + kBSubstep * s));
        const fp16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            (OPL_LDS fp16x4*)(st + b_lane[t] + kBSubstep * s + 4 * Cfg::kBRowBytes));
        half8 b;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          b[e] = lo[e];
          b[4 + e] = hi[e];
        }
        f.b[t] = b;
      } else {
        const OPL_LDS unsigned char* bb =
            (const OPL_LDS unsigned char*)(st + b_lane[t]) + kBSubstep * s;
        floatx4 b;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          b[e] = *(const OPL_LDS float*)(bb + e * Cfg::kBRowBytes);
        f.b[t] = b;
      }
    }
#pragma unroll
    for (int t = 1; t < kFM; ++t) load_a(st, s, f, t);
  };
  // fp32: the four k MFMAs of a block are kFM * kFN MFMAs apart.
  auto mma = [&](const Fragments<Cfg>& f) {
    if constexpr (kSize == 2) {
#pragma unroll
      for (int ti = 0; ti < kFM; ++ti)
#pragma unroll
        for (int tj = 0; tj < kFN; ++tj)
          acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              f.a[ti], f.b[tj], acc[ti][tj], 0, 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int ti = 0; ti < kFM; ++ti)
#pragma unroll
          for (int tj = 0; tj < kFN; ++tj)
            acc[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                f.a[ti][e], f.b[tj][e], acc[ti][tj], 0, 0, 0);
    }
  };
  // Scheduling groups for one substep: each block's MFMAs (one fp16 MFMA,
  // four fp32 ones) followed by their share of the LDS reads (the next
  // substep's fragments) and, with_dma, of the DMA issues, spread evenly,
  // so reads and copies issue in the MFMAs' shadow instead of in a burst.
  // (fp32 groups of single MFMAs left 29 VGPRs spilled: the scheduler then
  // stretched the accumulators' live ranges.)
  constexpr int kGroups = kFM * kFN;
  static_assert(2 * kGroups >= kReads && kGroups >= kIssues,
                "at most two reads and one copy per group");
  auto interleave = [&](bool with_dma) {
#pragma unroll
    for (int i = 0; i < kGroups; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, E::kMfmas, 0);  // MFMA
      const int reads = (i + 1) * kReads / kGroups - i * kReads / kGroups;
      if (reads >= 1) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if (reads >= 2) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (with_dma && (i + 1) * kIssues / kGroups != i * kIssues / kGroups)
        __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);  // VMEM
    }
  };
  // s_waitcnt vmcnt(n) expcnt(7) lgkmcnt(0): this wave's LDS reads and all
  // but its newest n DMA copies are complete. The release fence of
  // __syncthreads() does not wait for the copies, so the wait is explicit
  // and the barrier bare.
  auto wait_copies = [](auto outstanding) {
    constexpr int n = decltype(outstanding)::value;
    static_assert(n < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | 0x70);
  };
  // Every wave's copies of all but the newest kStages - 2 steps have landed
  // and no wave still reads the stage to be refilled.
  auto sync_stage = [&] {
    wait_copies(std::integral_constant<int, (Cfg::kStages - 2) * kIssues>());
    asm volatile("s_barrier" ::: "memory");
  };

  // A tail part writes its whole tile, row-major, to its partial slot;
  // sum_tail_kernel adds the parts in split order.
  float* const out = split >= 0
      ? tail.partial + static_cast<std::size_t>(split * tail.tiles + tail_index) * kBM * kBN
      : C + static_cast<std::size_t>(m0) * N + n0;
  const int ldo = split >= 0 ? kBN : N;
  // (a part's rows past M are never summed, so they are not written)
  const int row_end = min(kBM, M - m0);
  const int col_end = split >= 0 ? kBN : N - n0;
  const bool full = row_end >= kBM && col_end >= kBN;
  // Whole fp16 tiles leave through LDS: each wavefront writes 32 rows of
  // its 128 x 64 (or 64 x 64) sub-tile at a time into its own 8.5 KiB
  // block (68-float rows: the accumulator layout's
  // four row groups of a write land on different banks, and rows stay
  // 16-byte aligned), then reads them back row-major and stores 16 bytes
  // per lane, four 256-byte row segments per instruction: 32 store
  // instructions per lane instead of 128 single-float ones, each writing
  // whole cache lines (which the non-temporal stores need). Measured on
  // MI355X (us, per-float -> staged, cached stores): 4096^3 106.8 -> 104.0,
  // 8192^3 866 -> 852, 8192^2 x 2048 241 -> 227, 8192^2 x 4096 424 -> 406,
  // 16384^2 x 4096 1906 -> 1811. (fp32 keeps the per-float stores: with
  // the staged ones its main loop compiled slower, 4096^3 923 -> 1242.)
  constexpr int kWaves = kWM * kWN;
  constexpr int kOutPitch = 68;                       // floats per staged row
  constexpr int kOutBlock = 32 * kOutPitch * 4;       // bytes per wavefront
  constexpr int kBlocksPerStage = kWaves / Cfg::kStages;  // wavefront blocks per stage array
  // (not the four-stage 256 x 256 instance, K % 64 == 32, which already
  // runs at the 256-VGPR limit)
  constexpr bool kStagedOut = kSize == 2 && kFN == 4 && kFM % 2 == 0 &&
                              (Cfg::kStages == 2 || kWaves == 4) &&
                              kWaves % Cfg::kStages == 0 &&
                              kBlocksPerStage * kOutBlock <= Cfg::kStage;
  // (any row length: the 16-byte stores need only 4-byte alignment under
  // the target's unaligned access mode)
  const bool staged = kStagedOut && full;
  // st: the stage arrays in order (the last two unused with two stages).
  auto store_staged = [&](unsigned char* s0, unsigned char* s1, unsigned char* s2,
                          unsigned char* s3) {
    // every wave's last reads and copies are done before any block is written
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("s_barrier" ::: "memory");
    const int array = wave / kBlocksPerStage;
    unsigned char* const base = array == 0 ? s0 : array == 1 ? s1 : array == 2 ? s2 : s3;
    OPL_LDS float* const blk =
        (OPL_LDS float*)(base + (wave % kBlocksPerStage) * kOutBlock);
    float* const wout = out + static_cast<std::size_t>(wm * (kBM / kWM)) * ldo + wn * (kBN / kWN);
#pragma unroll
    for (int q = 0; q < kFM / 2; ++q) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int tj = 0; tj < kFN; ++tj)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            blk[(16 * t + 4 * group + e) * kOutPitch + 16 * tj + gl] = acc[2 * q + t][tj][e];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = 4 * i + lane / 16;
        const int c4 = lane % 16;
        const floatx4 v = *(const OPL_LDS floatx4*)(blk + row * kOutPitch + 4 * c4);
        typedef float floatx4u __attribute__((ext_vector_type(4), aligned(4)));
        floatx4u* const p = reinterpret_cast<floatx4u*>(
            wout + static_cast<std::size_t>(32 * q + row) * ldo + 4 * c4);
        if constexpr (kStreamC)
          __builtin_nontemporal_store(v, p);
        else
          *p = v;
      }
    }
  };

  Fragments<Cfg> f0, f1;
  if constexpr (Cfg::kStages == 2) {
    __shared__ __attribute__((aligned(1024))) unsigned char stage0[Cfg::kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage1[Cfg::kStage];
    // Step `step` computes from `cur` (complete); `nxt` holds step + 1 (in
    // flight). Substep 0 reads substep 1's fragments from `cur` under its
    // MFMAs. Then every wave has finished reading `cur` and step + 1 has
    // landed (sync_stage), so substep 1 refills `cur` with step + 2 and
    // reads the next step's first fragments from `nxt` under its MFMAs: the
    // barrier never waits on an LDS read.
    // The second substep (copies, next fragments, MFMAs) runs at raised
    // wave priority: the waves that left the barrier first get their
    // copies and reads issued ahead of the SIMD's other wavefront. Measured
    // on MI355X (us, 8192^3 / 4096^3, two runs each): 883.0, 884.1 ->
    // 873.2, 869.8 / 107.1, 106.0 -> 105.2, 105.1; raising it for the first
    // substep instead was slower (896.1).
    auto tile = [&](unsigned char* cur, unsigned char* nxt, int step) {
      load(cur, 1, f1);
      mma(f0);
      interleave(false);
      __builtin_amdgcn_sched_barrier(0);
      sync_stage();
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      issue(cur, step + 2);
      load(nxt, 0, f0);
      mma(f1);
      interleave(true);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    };
    issue(stage0, 0);
    issue(stage1, 1);
    if (fix && threadIdx.x == 0) {
      end_elems[0] = a_end_value;
      end_elems[1] = b_end_value;
    }
    wait_copies(std::integral_constant<int, kIssues>());
    asm volatile("s_barrier" ::: "memory");
    if (fix) fix_stage(stage0);
    load(stage0, 0, f0);
    __builtin_amdgcn_sched_barrier(0);
    int step = 0;
    for (; step + 1 < steps; step += 2) {
      tile(stage0, stage1, step);
      tile(stage1, stage0, step + 1);
    }
    if (step < steps) tile(stage0, stage1, step);
    if constexpr (kStagedOut) {
      if (staged) {
        store_staged(stage0, stage1, stage0, stage1);
        return;
      }
    }
  } else {
    __shared__ __attribute__((aligned(1024))) unsigned char stage0[Cfg::kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage1[Cfg::kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage2[Cfg::kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage3[Cfg::kStage];
    // Step `step` computes from fragments already in registers (`cur`, read
    // from stage step % 4 during the previous step). At its top every wave
    // has finished reading stage step % 4 and step + 1 has landed
    // (sync_stage), so the step refills stage step % 4 with step + 4 and
    // reads step + 1's fragments from `next` under its MFMAs.
    auto tile = [&](unsigned char* refill, const unsigned char* next, int step,
                    const Fragments<Cfg>& cur, Fragments<Cfg>& nxt) {
      sync_stage();
      __builtin_amdgcn_sched_barrier(0);
      issue(refill, step + 4);
      load(next, 0, nxt);
      mma(cur);
      interleave(true);
      __builtin_amdgcn_sched_barrier(0);
    };
    issue(stage0, 0);
    issue(stage1, 1);
    issue(stage2, 2);
    issue(stage3, 3);
    if (fix && threadIdx.x == 0) {
      end_elems[0] = a_end_value;
      end_elems[1] = b_end_value;
    }
    wait_copies(std::integral_constant<int, 3 * kIssues>());
    asm volatile("s_barrier" ::: "memory");
    if (fix) fix_stage(stage0);
    load(stage0, 0, f0);
    __builtin_amdgcn_sched_barrier(0);
    int step = 0;
    for (; step + 4 <= steps; step += 4) {
      tile(stage0, stage1, step, f0, f1);
      tile(stage1, stage2, step + 1, f1, f0);
      tile(stage2, stage3, step + 2, f0, f1);
      tile(stage3, stage0, step + 3, f1, f0);
    }
    if (step < steps) tile(stage0, stage1, step, f0, f1);
    if (step + 1 < steps) tile(stage1, stage2, step + 1, f1, f0);
    if (step + 2 < steps) tile(stage2, stage3, step + 2, f0, f1);
    if constexpr (kStagedOut) {
      if (staged) {
        store_staged(stage0, stage1, stage2, stage3);
        return;
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the last (empty) copies

#pragma unroll
  for (int ti = 0; ti < kFM; ++ti) {
#pragma unroll
    for (int tj = 0; tj < kFN; ++tj) {
      const int col = wn * (kBN / kWN) + 16 * tj + gl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = wm * (kBM / kWM) + 16 * ti + 4 * group + e;
        if (full || (row < row_end && col < col_end)) {
          float* const p = out + static_cast<std::size_t>(row) * ldo + col;
          // (a compile-time choice: under a run-time branch the compiler
          // merges the two stores and drops the non-temporal hint)
          if constexpr (kStreamC)
            __builtin_nontemporal_store(acc[ti][tj][e], p);
          else
            *p = acc[ti][tj][e];
        }
      }
    }
  }
}

// C tiles of a split tail: the sum, in split order, of each tail tile's
// `splits` partial tiles. One float4 of a tile row per thread.
template <typename Cfg>
__global__ __launch_bounds__(256) void sum_tail_kernel(float* __restrict__ C, int M, int N,
                                                       TailSplit tail) {
  constexpr int kBM = Cfg::kBM, kBN = Cfg::kBN;
  const int tiles_m = (M + kBM - 1) / kBM;
  const int tiles_n = (N + kBN - 1) / kBN;
  const int t = blockIdx.y;  // tail tile
  const int q = blockIdx.x * 256 + threadIdx.x;  // float4 of the tile
  const int lr = q / (kBN / 4);
  const int lc = 4 * (q % (kBN / 4));
  int tm, tn;
  grouped_tile(tail.full_tiles + t, tiles_m, tiles_n, &tm, &tn);
  const int row = tm * kBM + lr;
  const int col = tn * kBN + lc;
  if (lr >= kBM || row >= M || col >= N) return;
  typedef float f4 __attribute__((ext_vector_type(4)));
  f4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int sp = 0; sp < tail.splits; ++sp) {
    const f4 v = *reinterpret_cast<const f4*>(
        tail.partial + static_cast<std::size_t>(sp * tail.tiles + t) * kBM * kBN +
        static_cast<std::size_t>(lr) * kBN + lc);
    sum += v;
  }
  float* const dst = C + static_cast<std::size_t>(row) * N + col;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (col + e < N) dst[e] = sum[e];
}

#undef OPL_LDS
}  // namespace dma

// ---------------------------------------------------------------------------
// Skinny GEMM, M <= 16 (the reference's M == 1 and M <= 16 configurations,
// src/gemm.cu:445-448 and :464-467; LLM decode shapes such as 1 x 4096 x
// 4096). The product is a stream over B (K x N): 2 MNK flops for 2-4 bytes
// of B per (k, n) pair, far below the matrix cores' balance, so the kernel
// is built to stream B at HBM rate with vector-ALU dot products:
//   * a 256-thread workgroup takes a 256-byte-wide column block of B (64
//     fp32 or 128 fp16 columns) and a chunk of K rows; 16 lanes cover one
//     row segment with 16-byte loads, 16 rows are in flight per step;
//   * the workgroup's A chunk is staged in LDS transposed ([k][m]), so a
//     lane reads the M values for its row with 16-byte LDS reads that all
//     16 lanes of the row share;
//   * fp16 multiplies pairs of rows with v_dot2_f32_f16 (two products per
//     instruction, fp32 accumulation), fp32 uses FMAs;
//   * partial sums reduce across the 4 lanes per wavefront that share a
//     column (lane shuffles), then across the 4 wavefronts through LDS, in
//     a fixed order;
//   * K is split over enough workgroups to fill the GPU; per-split partials
//     go to scratch (arena or workspace) and a second kernel sums them in split
//     order, so results are deterministic;
//   * from M = 5 (fp16) or 9 (fp32) the vector-ALU dot products cost more
//     than the B stream, and skinny_mfma_kernel (below) takes over.
namespace skinny {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMaxM = 16;  // the vector-ALU kernel's largest M
constexpr int kLanesPerRow = 16;                     // one 256-byte row segment
constexpr int kRowGroups = kThreads / kLanesPerRow;  // 16
constexpr int kWaves = kThreads / opl::kWaveSize;    // 4
constexpr int kMaxChunk = 512;                       // K rows per workgroup

template <typename T>
struct Cfg {
  static constexpr int kPerLane = 16 / sizeof(T);       // columns per lane
  static constexpr int kBlockN = kLanesPerRow * kPerLane;  // 64 fp32, 128 fp16
  static constexpr int kRowsPerStep = sizeof(T) == 2 ? 2 : 1;  // dot2 pairs
  // From this M on the matrix-core variant is faster (measured on MI355X,
  // N = K = 4096: fp16 M 4 -> 11.3 us vector ALU, M 6 -> 12.3 us matrix
  // cores; fp32 M 8 -> 18.7 / 20.6 us, M 12 -> 27.9 / 21.9 us).
  static constexpr int kMfmaMinM = sizeof(T) == 2 ? 5 : 9;
  // The matrix-core kernel's largest M: 2 row blocks of 16 (fp16) or 4
  // (fp32). Beyond, the 128 x 128-tile kernel split along K is faster.
  // Measured on MI355X, N = K = 4096 (us, skinny vs 128 x 128 tiles split
  // along K): fp16 M = 17 15.7 vs 19.6, M = 32 17.6 vs 20.8, M = 48 25.0
  // vs 21.9, M = 64 27.5 vs 23.1; fp32 M = 17 23.6 vs 43.3, M = 32 25.0 vs
  // 44.2, M = 48 41.1 vs 45.1, M = 64 42.1 vs 46.0.
  static constexpr int kMaxMfmaM = sizeof(T) == 2 ? 32 : 64;
};

// Row steps (16-byte loads of one or two rows) in flight per thread per
// batch, sized so accumulators (M x 4 or M x 8 floats) plus the batch stay
// within 256 VGPRs, i.e. at least two wavefronts per SIMD.
template <typename T, int M>
constexpr int batch_for() {
  return sizeof(T) == 2 ? (M <= 2 ? 8 : (M <= 4 ? 4 : 2)) : (M <= 4 ? 8 : 4);
}

// One 16-byte chunk of B (P columns of row r) and, for fp16, of row r + 1;
// rows at or past k_end read a valid row and are zeroed.
template <typename T>
struct RowChunk {
  using Vec = typename std::conditional<sizeof(T) == 2, half8, float4v>::type;
  Vec v[Cfg<T>::kRowsPerStep];
};

template <typename T>
__device__ __forceinline__ RowChunk<T> load_rows(const T* __restrict__ B, int n,
                                                 int col, int r, int k_end) {
  RowChunk<T> c;
#pragma unroll
  for (int s = 0; s < Cfg<T>::kRowsPerStep; ++s) {
    const int row = r + s;
    const int rc = row < k_end ? row : k_end - 1;
    using Vec = typename RowChunk<T>::Vec;
    // B is streamed once: non-temporal loads. Measured on MI355X (us, N = K
    // = 4096, cached -> non-temporal): fp16 M = 1 10.36 -> 9.70, M = 4
    // 11.84 -> 11.47; fp32 M = 1 15.73 -> 14.75, M = 8 18.33 -> 17.49.
    Vec v = __builtin_nontemporal_load(
        reinterpret_cast<const Vec*>(B + static_cast<std::size_t>(rc) * n + col));
    if (row >= k_end) {
#pragma unroll
      for (int j = 0; j < Cfg<T>::kPerLane; ++j) v[j] = T(0);
    }
    c.v[s] = v;
  }
  return c;
}

template <typename T, int M>
__device__ __forceinline__ void accumulate_rows(const RowChunk<T>& c,
                                                const float* ak,
                                                float (&acc)[M][Cfg<T>::kPerLane]) {
  constexpr int P = Cfg<T>::kPerLane;
  if constexpr (sizeof(T) == 2) {
    half2v bp[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
      bp[j][0] = c.v[0][j];
      bp[j][1] = c.v[1][j];
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const half2v a = __builtin_bit_cast(half2v, ak[m]);
#pragma unroll
      for (int j = 0; j < P; ++j)
        acc[m][j] = __builtin_amdgcn_fdot2(a, bp[j], acc[m][j], false);
    }
  } else {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float a = ak[m];
#pragma unroll
      for (int j = 0; j < P; ++j) acc[m][j] = fmaf(a, c.v[0][j], acc[m][j]);
    }
  }
}

template <typename T, int M>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void skinny_kernel(
    const T* __restrict__ A, const T* __restrict__ B, float* __restrict__ out,
    int m_rows, int n, int k, int chunk) {
  using C = Cfg<T>;
  constexpr int P = C::kPerLane;
  constexpr int R = C::kRowsPerStep;
  // A chunk, transposed: fp32 as [k][M]; fp16 as [k / 2][M] pairs (k, k+1).
  // One extra all-zero row (index kMaxChunk / R) absorbs batch steps past
  // the chunk.
  constexpr int kStage = (kMaxChunk / R + 1) * M;
  constexpr int kStagePerThread = (kStage + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) float a_lds[kStage];
  __shared__ float red[kWaves * M * C::kBlockN];

  constexpr int kBatch = batch_for<T, M>();
  const int n0 = blockIdx.x * C::kBlockN;
  const int k0 = blockIdx.y * chunk;
  const int k_end = min(k, k0 + chunk);
  const int steps = (k_end - k0 + R - 1) / R;  // rows (fp16: row pairs)
  const int tid = threadIdx.x;
  const int lane_col = tid % kLanesPerRow;
  const int group = tid / kLanesPerRow;
  // Columns past N: read a valid chunk (n % P == 0), results not stored.
  const int col = min(n0 + lane_col * P, n - P);

  // A values of this chunk (zeros past k_end and past m_rows) into
  // registers first, then the first batch of B rows, then A into LDS: the
  // B loads' latency overlaps the staging and its barrier.
  float a_reg[kStagePerThread];
#pragma unroll
  for (int s = 0; s < kStagePerThread; ++s) {
    const int i = tid + kThreads * s;
    const int kk = i / M;
    const int m = i % M;
    float v = 0.0f;
    if (i < chunk / R * M && m < m_rows) {
      if constexpr (R == 2) {
        half2v h;
        const int r = k0 + 2 * kk;
        h[0] = r < k_end ? A[static_cast<std::size_t>(m) * k + r] : T(0);
        h[1] = r + 1 < k_end ? A[static_cast<std::size_t>(m) * k + r + 1] : T(0);
        v = __builtin_bit_cast(float, h);
      } else {
        const int r = k0 + kk;
        v = r < k_end ? static_cast<float>(A[static_cast<std::size_t>(m) * k + r]) : 0.0f;
      }
    }
    a_reg[s] = v;
  }
  RowChunk<T> b[kBatch];
#pragma unroll
  for (int u = 0; u < kBatch; ++u)
    b[u] = load_rows<T>(B, n, col, k0 + R * (group + kRowGroups * u), k_end);
#pragma unroll
  for (int s = 0; s < kStagePerThread; ++s) {
    const int i = tid + kThreads * s;
    if (i < kStage) a_lds[i] = a_reg[s];
  }
  __syncthreads();

  float acc[M][P];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < P; ++j) acc[m][j] = 0.0f;

  for (int base = group;; base += kBatch * kRowGroups) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      // Steps past `steps` read zeroed B rows and zero A slots (staged as
      // zero past k_end, or the zero row past the chunk).
      const int kk = min(base + kRowGroups * u, kMaxChunk / R);
      accumulate_rows<T, M>(b[u], a_lds + kk * M, acc);
    }
    const int next = base + kBatch * kRowGroups;
    if (next >= steps) break;
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      b[u] = load_rows<T>(B, n, col, k0 + R * (next + kRowGroups * u), k_end);
  }

  // Lanes l, l^16, l^32, l^48 of a wavefront share a column chunk.
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < P; ++j) {
      float v = acc[m][j];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      acc[m][j] = v;
    }
  const int wave = tid / opl::kWaveSize;
  const int lane = tid % opl::kWaveSize;
  if (lane < kLanesPerRow) {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < P; ++j)
        red[(wave * M + m) * C::kBlockN + lane * P + j] = acc[m][j];
  }
  __syncthreads();
  float* dst = out + static_cast<std::size_t>(blockIdx.y) * m_rows * n;
  for (int i = tid; i < M * C::kBlockN; i += kThreads) {
    const int m = i / C::kBlockN;
    const int c = i % C::kBlockN;
    if (m < m_rows && n0 + c < n) {
      float s = red[m * C::kBlockN + c];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) s += red[(w * M + m) * C::kBlockN + c];
      dst[static_cast<std::size_t>(m) * n + n0 + c] = s;
    }
  }
}

// Matrix-core variant for larger M (up to 32 fp16, 64 fp32, in row blocks
// of 16): one v_mfma_f32_16x16x16_f16 (fp16) or v_mfma_f32_16x16x4_f32
// (fp32) turns 16 rows of A times a 16 x 16 block of B into a 16 x 16 block
// of C, where the vector-ALU kernel spends one dot product per (m, column
// pair) and becomes ALU-bound as M grows.
// B is never transposed: the MFMA only needs A and B to agree on which k
// fills each of its k slots. K is walked in blocks of 16 rows; lane (g, c)
// (g = lane / 16, c = lane % 16) owns rows 4g .. 4g+3 of each block (fp32
// with unaligned A: blocks of 4 rows, row g each, 16 blocks in flight, as
// the element loads gain nothing from the grouping):
//   * it loads a 16-byte chunk (columns P*c .. P*c+P-1) of each of those
//     rows, and MFMA j takes column j of every lane's chunk, so tile column
//     c of MFMA j is matrix column P*c + j and P MFMAs cover the
//     workgroup's 16 P columns;
//   * its A operand values A[c][4g .. 4g+3] are contiguous, one 8-byte
//     (fp16) or 16-byte (fp32) load straight from global memory (A is
//     L2-resident), issued with the B loads, so nothing waits on a staging
//     barrier; rows that are not 4-aligned fall back to element loads;
//   * fp16 feeds the four rows to one 16x16x16 MFMA (k slots 4g .. 4g+3);
//     fp32 issues four 16x16x4 MFMAs, the u-th taking row 4g + u in k slot
//     g.
// Splits, the workgroup shape and the partial sums are those of
// skinny_kernel.
template <typename T>
struct MfmaCfg;
template <>
struct MfmaCfg<_Float16> {
  typedef _Float16 AOp __attribute__((ext_vector_type(4)));
  typedef _Float16 AVec __attribute__((ext_vector_type(4)));
  static constexpr int kBatch = 4;    // 16-row k blocks in flight per wavefront
  __device__ static floatx4v mma(AOp a, AOp b, floatx4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct MfmaCfg<float> {
  typedef float AOp;
  typedef float AVec __attribute__((ext_vector_type(4)));
  static constexpr int kBatch = 4;
  __device__ static floatx4v mma(AOp a, AOp b, floatx4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

// Rows of a k block that one lane owns (and the MFMA k slots they fill).
constexpr int kLaneRows = 4;

// kVecA: K % 4 == 0 and A aligned to 4 elements, so each lane's four A
// values of a block are one aligned vector, wholly inside or outside k_end.
// kMB row blocks of 16 (M up to 16 kMB): every B chunk a lane loads feeds
// one MFMA per row block, so B is still streamed once.
template <typename T, bool kVecA, int kMB>
__global__ __launch_bounds__(kThreads) void skinny_mfma_kernel(
    const T* __restrict__ A, const T* __restrict__ B, float* __restrict__ out,
    int m_rows, int n, int k, int chunk) {
  using MC = MfmaCfg<T>;
  using Vec = typename RowChunk<T>::Vec;  // one 16-byte chunk of a B row
  constexpr int P = Cfg<T>::kPerLane;     // columns per lane
  constexpr int BN = Cfg<T>::kBlockN;     // 16 * P
  // Rows per lane and k block: 4, or 1 for fp32 without vector A loads.
  constexpr int R = sizeof(T) == 4 && !kVecA ? 1 : kLaneRows;
  constexpr int KB = 4 * R;  // rows per k block
  // k blocks in flight, halved at four row blocks (fp32 only): the full
  // batch compiled to 193 VGPRs there, one wavefront per SIMD, the half to
  // 78
  constexpr int kBatch = (R == 1 ? 16 : MC::kBatch) / (kMB >= 4 ? 2 : 1);
  using AVec = typename std::conditional<R == 1, T, typename MC::AVec>::type;
  // k slot q of a lane's A values
  auto a_at = [](const AVec& a, int q) -> T {
    if constexpr (R == 1) return a; else return a[q];
  };
  __shared__ float red[kWaves * opl::kWaveSize * P * 4];

  const int n0 = blockIdx.x * BN;
  const int k0 = blockIdx.y * chunk;
  const int k_end = min(k, k0 + chunk);
  const int tid = threadIdx.x;
  const int lane = tid % opl::kWaveSize;
  const int wave = tid / opl::kWaveSize;
  const int g = lane / 16;
  const int c = lane % 16;
  // Columns past N: read a valid chunk (n % P == 0), results not stored.
  const int col = min(n0 + c * P, n - P);
  const int blocks = (k_end - k0 + KB - 1) / KB;

  // k block b, lane group g: k rows k0 + KB b + R g + q (q < R). B: a
  // 16-byte chunk of each row; A: A[16 mb + c][row] of each row block mb
  // (read from L2, every workgroup of the split reads the same A). Rows
  // past k_end read valid memory and are zeroed, as are A rows past m_rows.
  auto load_block = [&](int b, Vec (&v)[R], AVec (&a)[kMB]) {
    const int r0 = k0 + KB * b + R * g;
#pragma unroll
    for (int q = 0; q < R; ++q) {
      const int r = r0 + q;
      const bool in = r < k_end;
      const int rc = in ? r : k_end - 1;
      // Non-temporal B loads for fp32 only. Measured on MI355X (us, cached
      // -> non-temporal): fp32 M = 16 20.07 -> 19.51, M = 64 41.98 ->
      // 41.24; fp16 M = 16 13.53 -> 14.04, M = 32 17.91 -> 19.58 (N = K =
      // 4096).
      const Vec* const src = reinterpret_cast<const Vec*>(B + static_cast<std::size_t>(rc) * n + col);
      Vec x;
      if constexpr (sizeof(T) == 4)
        x = __builtin_nontemporal_load(src);
      else
        x = *src;
#pragma unroll
      for (int j = 0; j < P; ++j) x[j] = in ? x[j] : T(0);
      v[q] = x;
      if constexpr (!kVecA) {
        // element loads, each issued beside its B row's load
#pragma unroll
        for (int mb = 0; mb < kMB; ++mb) {
          const int arow = 16 * mb + c;
          const bool a_in = in && arow < m_rows;
          const T av = A[a_in ? static_cast<std::size_t>(arow) * k + r : 0];
          if constexpr (R == 1)
            a[mb] = a_in ? av : T(0);
          else
            a[mb][q] = a_in ? av : T(0);
        }
      }
    }
    if constexpr (kVecA) {
      // r0 % 4 == 0 and k_end % 4 == 0: rows r0 .. r0+3 are all in or all
      // out. Out-of-range lanes read A[0 .. 3] (k >= 4) and zero it.
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        const int arow = 16 * mb + c;
        const bool a_in = r0 < k_end && arow < m_rows;
        AVec x = *reinterpret_cast<const AVec*>(
            A + (a_in ? static_cast<std::size_t>(arow) * k + r0 : 0));
#pragma unroll
        for (int q = 0; q < R; ++q) a[mb][q] = a_in ? x[q] : T(0);
      }
    }
  };

  floatx4v acc[kMB][P];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int j = 0; j < P; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[mb][j][e] = 0.0f;

  Vec v[kBatch][R];
  AVec a[kBatch][kMB];
  for (int b0 = wave; b0 < blocks; b0 += kWaves * kBatch) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int b = b0 + kWaves * u;
      load_block(b < blocks ? b : blocks - 1, v[u], a[u]);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (b0 + kWaves * u < blocks) {  // wave-uniform
#pragma unroll
        for (int j = 0; j < P; ++j) {
          if constexpr (sizeof(T) == 2) {
            typename MC::AOp bop;
#pragma unroll
            for (int q = 0; q < R; ++q) bop[q] = v[u][q][j];
#pragma unroll
            for (int mb = 0; mb < kMB; ++mb) acc[mb][j] = MC::mma(a[u][mb], bop, acc[mb][j]);
          } else {
#pragma unroll
            for (int q = 0; q < R; ++q)
#pragma unroll
              for (int mb = 0; mb < kMB; ++mb)
                acc[mb][j] = MC::mma(a_at(a[u][mb], q), v[u][q][j], acc[mb][j]);
          }
        }
      }
    }
  }

  // acc[mb][j][i] = C[16 mb + 4 g + i][n0 + P c + j] of this wavefront's
  // k blocks; the wavefronts' sums go through LDS one row block at a time.
  float* dst = out + static_cast<std::size_t>(blockIdx.y) * m_rows * n;
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb) {
    if (mb > 0) __syncthreads();  // the previous block's reads are done
#pragma unroll
    for (int j = 0; j < P; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[((wave * opl::kWaveSize + lane) * P + j) * 4 + i] = acc[mb][j][i];
    __syncthreads();
    for (int o = tid; o < 16 * BN; o += kThreads) {
      const int m = o / BN;
      const int co = o % BN;
      const int row = 16 * mb + m;
      if (row < m_rows && n0 + co < n) {
        const int src = ((16 * (m / 4) + co / P) * P + co % P) * 4 + m % 4;
        float s = red[src];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) s += red[w * opl::kWaveSize * P * 4 + src];
        dst[static_cast<std::size_t>(row) * n + n0 + co] = s;
      }
    }
  }
}

// out[i] = sum over splits s (in order) of part[s][i]. Each thread issues
// the loads of up to kSplitBatch splits before adding them, so a sum costs
// one memory round trip per batch instead of one per split.
constexpr int kSplitBatch = 16;
constexpr int kSumThreads = 64;

__global__ __launch_bounds__(kSumThreads) void sum_splits_kernel(
    const float* __restrict__ part, float* __restrict__ out, long long count,
    int splits) {
  for (long long i = blockIdx.x * static_cast<long long>(kSumThreads) + threadIdx.x;
       i < count; i += static_cast<long long>(gridDim.x) * kSumThreads) {
    float s = part[i];
    for (int p0 = 1; p0 < splits; p0 += kSplitBatch) {
      float v[kSplitBatch];
#pragma unroll
      for (int u = 0; u < kSplitBatch; ++u) {
        const int p = min(p0 + u, splits - 1);  // in range; extra slots unused
        v[u] = part[p * count + i];
      }
#pragma unroll
      for (int u = 0; u < kSplitBatch; ++u)
        if (p0 + u < splits) s += v[u];
    }
    out[i] = s;
  }
}

template <typename T, int M>
void launch_m(const T* a, const T* b, float* dst, int m, int n, int k,
              int chunk, dim3 grid, hipStream_t stream) {
  skinny_kernel<T, M><<<grid, dim3(kThreads), 0, stream>>>(a, b, dst, m, n, k, chunk);
}

template <typename T, int kMB>
void launch_mfma(bool vec_a, const T* a, const T* b, float* dst, int m, int n, int k,
                 int chunk, dim3 grid, hipStream_t stream) {
  if (vec_a)
    skinny_mfma_kernel<T, true, kMB><<<grid, dim3(kThreads), 0, stream>>>(a, b, dst, m, n, k,
                                                                        chunk);
  else
    skinny_mfma_kernel<T, false, kMB><<<grid, dim3(kThreads), 0, stream>>>(a, b, dst, m, n, k,
                                                                         chunk);
}

template <typename T>
bool applies(const T* b, int m, int n) {
  return m <= Cfg<T>::kMaxMfmaM && n % Cfg<T>::kPerLane == 0 && opl::aligned16(b);
}

// K split of one call: `splits` workgroup rows of `chunk` K rows each (a
// multiple of 32, at most kMaxChunk, the A rows one workgroup stages), and
// the scratch bytes of their partial sums (0 for one split).
struct Plan {
  int splits = 1;
  int chunk = 0;
  std::size_t bytes = 0;
  bool ok = false;  // false: no split fits `capacity`
};

inline Plan plan_with(int m, int n, int k, int splits) {
  Plan p;
  int chunk = (k + splits - 1) / splits;
  chunk = (chunk + 31) / 32 * 32;
  if (chunk > kMaxChunk) chunk = kMaxChunk;
  p.chunk = chunk;
  p.splits = (k + chunk - 1) / chunk;
  p.bytes = p.splits > 1 ? static_cast<std::size_t>(p.splits) * m * n * sizeof(float) : 0;
  p.ok = true;
  return p;
}

// Enough workgroups to cover the GPU about twice, as scratch allows: fewer
// splits when their partials would not fit `capacity`, none of this kernel
// when even the fewest (K / kMaxChunk) would not.
template <typename T>
Plan plan(int m, int n, int k, std::size_t capacity) {
  const int blocks_n = (n + Cfg<T>::kBlockN - 1) / Cfg<T>::kBlockN;
  int splits = (512 + blocks_n - 1) / blocks_n;
  const int max_splits = (k + 63) / 64;
  if (splits > max_splits) splits = max_splits;
  if (splits < 1) splits = 1;
  Plan p = plan_with(m, n, k, splits);
  if (p.bytes <= capacity) return p;
  const std::size_t per_split = static_cast<std::size_t>(m) * n * sizeof(float);
  const std::size_t fit = capacity / per_split;
  const int fewest = (k + kMaxChunk - 1) / kMaxChunk;
  if (fit < static_cast<std::size_t>(fewest)) return Plan{};
  p = plan_with(m, n, k, static_cast<int>(fit < static_cast<std::size_t>(splits) ? fit : splits));
  p.ok = p.bytes <= capacity;
  return p;
}

// Runs plan `p` (p.ok); `partials` holds p.bytes of scratch when p.splits > 1.
template <typename T>
hipError_t launch(const T* a, const T* b, float* c, int m, int n, int k, const Plan& p,
                  void* partials, opl::ScratchLease* lease, hipStream_t stream) {
  using C = Cfg<T>;
  const int blocks_n = (n + C::kBlockN - 1) / C::kBlockN;
  float* dst = p.splits > 1 ? static_cast<float*>(partials) : c;
  const int chunk = p.chunk;
  const dim3 grid(static_cast<unsigned>(blocks_n), static_cast<unsigned>(p.splits));
  if (m >= C::kMfmaMinM) {
    const bool vec_a =
        k % kLaneRows == 0 &&
        reinterpret_cast<std::uintptr_t>(a) % (kLaneRows * sizeof(T)) == 0;
    if (m <= 16) {
      launch_mfma<T, 1>(vec_a, a, b, dst, m, n, k, chunk, grid, stream);
    } else if (m <= 32) {
      launch_mfma<T, 2>(vec_a, a, b, dst, m, n, k, chunk, grid, stream);
    } else {
      if constexpr (C::kMaxMfmaM > 32)
        launch_mfma<T, 4>(vec_a, a, b, dst, m, n, k, chunk, grid, stream);
    }
  } else if (m == 1) launch_m<T, 1>(a, b, dst, m, n, k, chunk, grid, stream);
  else if (m <= 2) launch_m<T, 2>(a, b, dst, m, n, k, chunk, grid, stream);
  else if (m <= 4) launch_m<T, 4>(a, b, dst, m, n, k, chunk, grid, stream);
  else if (m <= 8) launch_m<T, 8>(a, b, dst, m, n, k, chunk, grid, stream);
  else launch_m<T, 16>(a, b, dst, m, n, k, chunk, grid, stream);
  if (p.splits > 1) {
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) return status;
    const long long count = static_cast<long long>(m) * n;
    const long long blocks = (count + kSumThreads - 1) / kSumThreads;
    return lease->launch_last(sum_splits_kernel,
                              dim3(static_cast<unsigned>(blocks < 16384 ? blocks : 16384)),
                              dim3(kSumThreads), static_cast<const float*>(dst), c, count,
                              p.splits);
  }
  return hipGetLastError();
}

}  // namespace skinny

// ---------------------------------------------------------------------------
// Narrow N (N <= 16: matrix-vector products and a few right-hand columns)
// for M past the skinny kernels: an HBM stream over A, which the tiled
// kernels would multiply in 128- or 256-column tiles of mostly padding.
// Each wavefront owns kRows consecutive rows of A; in every step of K lane
// l reads 16-byte chunk l of the step's 64 chunks from each of its rows,
// and the matching E x N block of B (rows k .. k + E - 1, all N columns,
// contiguous in row-major B: N aligned 16-byte loads, from L2, shared by
// the wavefront's rows). fp16 multiplies k pairs with v_dot2_f32_f16,
// fp32 with FMAs, into fp32 partials that are summed over the wavefront
// in a fixed order at the end. No scratch, one launch.
// ---------------------------------------------------------------------------
namespace narrow {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / opl::kWaveSize;
constexpr int kRows = 4;   // rows of A per wavefront
constexpr int kMaxN = 16;

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

template <typename T, int N>
__global__ __launch_bounds__(kThreads) void narrow_kernel(const T* __restrict__ A,
                                                          const T* __restrict__ B,
                                                          float* __restrict__ C, int M,
                                                          int K) {
  using Vec = typename std::conditional<sizeof(T) == 2, half8, float4v>::type;
  constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements per chunk
  constexpr int kUnroll = N <= 4 ? 2 : 1;               // K steps in flight
  const int lane = threadIdx.x % opl::kWaveSize;
  const int wave = threadIdx.x / opl::kWaveSize;
  const long long row0 =
      (static_cast<long long>(blockIdx.x) * kWaves + wave) * kRows;  // wave-uniform
  if (row0 >= M) return;  // no barrier follows
  const T* arow[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
    arow[r] = A + static_cast<std::size_t>(min(row0 + r, static_cast<long long>(M) - 1)) * K;
  float acc[kRows][N];
#pragma unroll
  for (int r = 0; r < kRows; ++r)
#pragma unroll
    for (int n = 0; n < N; ++n) acc[r][n] = 0.0f;

  const int chunks = K / E;  // K % E == 0
  for (int c0 = 0; c0 < chunks; c0 += opl::kWaveSize * kUnroll) {
    Vec a[kUnroll][kRows];
    Vec b[kUnroll][N];  // b[u][j]: elements E j .. E j + E - 1 of the E x N block
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = c0 + opl::kWaveSize * u + lane;
      const bool in = c < chunks;
      const int cc = in ? c : 0;
#pragma unroll
      for (int r = 0; r < kRows; ++r)
        // A is streamed once: non-temporal loads (MI355X, us, cached ->
        // non-temporal: fp16 4096 x 1 x 4096 8.62 -> 8.19, 4096 x 16 x 4096
        // 22.88 -> 22.49; fp32 4096 x 1 x 4096 17.23 -> 16.93)
        a[u][r] = __builtin_nontemporal_load(
            reinterpret_cast<const Vec*>(arow[r] + static_cast<std::size_t>(cc) * E));
      const T* bblk = B + static_cast<std::size_t>(cc) * E * N;
#pragma unroll
      for (int j = 0; j < N; ++j) b[u][j] = *reinterpret_cast<const Vec*>(bblk + E * j);
      if (!in) {
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
          for (int e = 0; e < E; ++e) a[u][r][e] = T(0);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      // B element (e, n) of the block is b[u][(e N + n) / E][(e N + n) % E].
      auto belem = [&](int e, int n) -> T {
        const int i = e * N + n;
        return b[u][i / E][i % E];
      };
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int e = 0; e < E; e += 2) {
#pragma unroll
          for (int n = 0; n < N; ++n) {
            half2v bp;
            bp[0] = belem(e, n);
            bp[1] = belem(e + 1, n);
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
              half2v ap;
              ap[0] = a[u][r][e];
              ap[1] = a[u][r][e + 1];
              acc[r][n] = __builtin_amdgcn_fdot2(ap, bp, acc[r][n], false);
            }
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
#pragma unroll
          for (int n = 0; n < N; ++n)
#pragma unroll
            for (int r = 0; r < kRows; ++r) acc[r][n] = fmaf(a[u][r][e], belem(e, n), acc[r][n]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const float v = opl::wave_reduce<opl::SumOp>(acc[r][n]);
      if (lane == 0 && row0 + r < M) C[static_cast<std::size_t>(row0 + r) * N + n] = v;
    }
  }
}

template <typename T>
bool applies(const T* a, const T* b, int n, int k) {
  constexpr int E = 16 / static_cast<int>(sizeof(T));
  return n <= kMaxN && k % E == 0 && opl::aligned16(a) && opl::aligned16(b);
}

template <typename T, int N>
hipError_t launch_n(const T* a, const T* b, float* c, int m, int k, hipStream_t stream) {
  const long long rows_per_block = static_cast<long long>(kWaves) * kRows;
  const long long blocks = (m + rows_per_block - 1) / rows_per_block;
  narrow_kernel<T, N><<<dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream>>>(
      a, b, c, m, k);
  return hipGetLastError();
}

template <typename T, int N = 1>
hipError_t launch(const T* a, const T* b, float* c, int m, int n, int k, hipStream_t stream) {
  if constexpr (N < kMaxN) {
    if (n != N) return launch<T, N + 1>(a, b, c, m, n, k, stream);
  }
  return launch_n<T, N>(a, b, c, m, k, stream);
}

}  // namespace narrow

typedef unsigned uint4v __attribute__((ext_vector_type(4)));

// The 16 bytes at p (any 2-byte alignment) from the aligned 16-byte
// chunk(s) covering them: word i of the result is bytes sh + 4i .. sh + 4i
// + 3 of the two chunks, sh = p mod 16, taken with v_alignbyte. Both chunks
// hold bytes of [p, p + 16), so they lie in pages those bytes occupy.
__device__ __forceinline__ uint4v load16_shifted(const void* p) {
  const std::uintptr_t addr = reinterpret_cast<std::uintptr_t>(p);
  const int sh = static_cast<int>(addr & 15);
  const uint4v* a = reinterpret_cast<const uint4v*>(addr - sh);
  const uint4v lo = a[0];
  if (sh == 0) return lo;
  const uint4v hi = a[1];
  const unsigned bs = static_cast<unsigned>(sh & 3);
  auto ab = [&](unsigned h, unsigned l) { return __builtin_amdgcn_alignbyte(h, l, bs); };
  uint4v out;
  switch (sh >> 2) {  // first source word; uniform across a row's chunks
    case 0: out = uint4v{ab(lo[1], lo[0]), ab(lo[2], lo[1]), ab(lo[3], lo[2]), ab(hi[0], lo[3])}; break;
    case 1: out = uint4v{ab(lo[2], lo[1]), ab(lo[3], lo[2]), ab(hi[0], lo[3]), ab(hi[1], hi[0])}; break;
    case 2: out = uint4v{ab(lo[3], lo[2]), ab(hi[0], lo[3]), ab(hi[1], hi[0]), ab(hi[2], hi[1])}; break;
    default: out = uint4v{ab(hi[0], lo[3]), ab(hi[1], hi[0]), ab(hi[2], hi[1]), ab(hi[3], hi[2])}; break;
  }
  return out;
}

// Copies a row-major fp16 [rows, cols] matrix into a zero-padded row-major
// [rows_p, cols_p] one whose rows are whole 16-byte chunks (cols_p a
// multiple of 8, 16-byte aligned destination): each thread writes whole
// chunks. A chunk whose source elements all exist is read as 16 bytes from
// the aligned chunk(s) covering it (the rows of an odd-width matrix start
// at every 2-byte phase); a row's last chunk and the padding rows go
// element by element.
__global__ __launch_bounds__(256) void pad_copy_kernel(const _Float16* __restrict__ src,
                                                       int rows, int cols,
                                                       _Float16* __restrict__ dst,
                                                       int rows_p, int cols_p) {
  using Chunk = Precision<_Float16>::Chunk;
  constexpr int E = Precision<_Float16>::kChunkElems;
  const long long per_row = cols_p / E;
  const long long total = static_cast<long long>(rows_p) * per_row;
  for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
       i < total; i += static_cast<long long>(gridDim.x) * blockDim.x) {
    const int r = static_cast<int>(i / per_row);
    const int c0 = static_cast<int>(i % per_row) * E;
    const _Float16* s = src + static_cast<std::size_t>(r) * cols;
    Chunk v;
    if (r < rows && c0 + E <= cols) {
      v = __builtin_bit_cast(Chunk, load16_shifted(s + c0));
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e)
        v[e] = (r < rows && c0 + e < cols) ? s[c0 + e] : _Float16(0);
    }
    *reinterpret_cast<Chunk*>(dst + static_cast<std::size_t>(r) * cols_p + c0) = v;
  }
}

void launch_pad_copy(const _Float16* src, int rows, int cols, _Float16* dst, int rows_p,
                     int cols_p, hipStream_t stream) {
  const long long chunks = static_cast<long long>(rows_p) * (cols_p / 8);
  const long long blocks = (chunks + 255) / 256;
  pad_copy_kernel<<<dim3(static_cast<unsigned>(blocks < 8192 ? blocks : 8192)), dim3(256), 0,
                    stream>>>(src, rows, cols, dst, rows_p, cols_p);
}

inline long long round_up(long long x, long long to) { return (x + to - 1) / to * to; }

// The direct-to-LDS kernel reads every operand in place, but fp16 rows
// that are not 4-byte aligned (odd K for A, odd N for B, or a base off a
// 4-byte boundary) start their 16-byte copies at a 2-byte phase, and those
// copies cost it time; dword-aligned rows cost nothing. Measured on MI355X
// (us, kernel alone): 4095^3 132 against 107 for the same grid aligned,
// 4097 x 4095 x 4093 150 against 119; 4096^3 with every row of A and B at
// a 2-byte phase 155 against 113, A only 126, B only 123; odd K only 119,
// odd N only 113; 8192 x 8191 x 8191 1106 against 871, odd K only 1046,
// odd N only 968. Dword-aligned: fp16 K = 4094 111, fp32 4095^3 928
// against 926. Large products therefore first copy such operands into
// rows padded to a whole number of chunks (about 11.5 us per 4095^2
// operand). Which ones, measured interleaved (us, median; nothing / A / B
// / both copied): 4095^3 131.3 / 126.1 / 128.1 / 131.3, 4097 x 4095 x
// 4093 149.1 / 144.8 / 145.9 / 148.2, 8192 x 8191 x 8191 1104 / 992 /
// 1044 / 932. So with both off: A alone from 10^11 flop (about 3700^3),
// both from 4 * 10^11 (about 5800^3); one operand off: that one from
// 2.75 * 10^11 (about 5200^3). A single copy pads its rows only (A [M,
// round_up(K, 8)], B [K, round_up(N, 8)]) and the kernel repairs K's last
// step itself; two copies are also padded along K to a multiple of 64 (A
// [M, K'], B [K', N'], zeros past K), and the kernel runs its plain
// schedule.
struct PadPlan {
  bool pad_a = false, pad_b = false;
  int k = 0;             // the K the kernel runs with
  int lda = 0, ldb = 0;  // row strides it reads with
  std::size_t a_bytes = 0, b_bytes = 0;  // each rounded to 256 bytes
  std::size_t bytes() const { return a_bytes + b_bytes; }
};

template <typename T>
PadPlan pad_plan(const T* a, const T* b, int m, int n, int k) {
  PadPlan p;
  p.k = k;
  p.lda = k;
  p.ldb = n;
  if constexpr (sizeof(T) == 2) {
    auto dword = [](const void* q) { return (reinterpret_cast<std::uintptr_t>(q) & 3u) == 0; };
    const bool off_a = k % 2 != 0 || !dword(a);
    const bool off_b = n % 2 != 0 || !dword(b);
    const double flops = 2.0 * m * n * static_cast<double>(k);
    bool pad_a = false, pad_b = false;
    if (off_a && off_b) {
      pad_a = flops >= 1.0e11;
      pad_b = flops >= 4.0e11;
    } else {
      pad_a = off_a && flops >= 2.75e11;
      pad_b = off_b && flops >= 2.75e11;
    }
    if (!pad_a && !pad_b) return p;
    const long long kk = pad_a && pad_b ? round_up(k, 64) : k;  // K the kernel runs with
    const long long kp = round_up(kk, 8), np = round_up(n, 8);
    if (kp > 0x7fffffffLL || np > 0x7fffffffLL) return p;
    p.pad_a = pad_a;
    p.pad_b = pad_b;
    p.k = static_cast<int>(kk);
    if (p.pad_a) {
      p.lda = static_cast<int>(kp);
      p.a_bytes = static_cast<std::size_t>(round_up(static_cast<long long>(m) * kp * 2, 256));
    }
    if (p.pad_b) {
      p.ldb = static_cast<int>(np);
      p.b_bytes = static_cast<std::size_t>(round_up(kk * np * 2, 256));
    }
  }
  return p;
}

// One launch of gemm_mfma_kernel with tile layout L and staging `staging`.
template <typename T, typename L>
hipError_t launch_generic(int staging, const T* a, const T* b, float* c, int m,
                          int n, int k, int ldb, hipStream_t stream) {
  const long long tiles = static_cast<long long>((m + L::kBM - 1) / L::kBM) *
                          ((n + L::kBN - 1) / L::kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(tiles)), block(L::kThreads);
  if (staging == kAligned16)
    gemm_mfma_kernel<T, kAligned16, L><<<grid, block, 0, stream>>>(a, b, c, m, n, k, ldb);
  else if (staging == kDword)
    gemm_mfma_kernel<T, kDword, L><<<grid, block, 0, stream>>>(a, b, c, m, n, k, ldb);
  else
    gemm_mfma_kernel<T, kElementwise, L><<<grid, block, 0, stream>>>(a, b, c, m, n, k, ldb);
  return hipGetLastError();
}

// fp32 grids of fewer 256 x 256 tiles than this run on 128 x 128 tiles: a
// 256 x 256 workgroup takes a whole CU for ~1 ms at K = 4096 whatever the
// grid, so below one tile per CU the smaller tiles win. Measured on MI355X
// (us, 256 x 256 vs 128 x 128): 1000 x 4096 x 4096 (64 tiles) 1006 vs 302;
// 2048 x 4096 x 4096 (128) 1007 vs 547; 3072 x 4096 x 4096 (192) 1009 vs
// 830; 4096^3 (256) 1010 vs 1078.
constexpr long long kSmallGridTilesF32 = 256;

template <typename T>
hipError_t launch_generic_for(int staging, const T* a, const T* b, float* c, int m,
                              int n, int k, int ldb, hipStream_t stream) {
  using L = typename LayoutFor<T>::type;
  if constexpr (std::is_same<T, float>::value) {
    const long long big_tiles = static_cast<long long>((m + L::kBM - 1) / L::kBM) *
                                ((n + L::kBN - 1) / L::kBN);
    if (big_tiles < kSmallGridTilesF32)
      return launch_generic<T, F32SmallLayout>(staging, a, b, c, m, n, k, ldb, stream);
  }
  return launch_generic<T, L>(staging, a, b, c, m, n, k, ldb, stream);
}

// The fastest staging the operands allow (Staging above).
template <typename T>
int staging_for(const T* a, const T* b, int n, int k) {
  constexpr int E = Precision<T>::kChunkElems;
  if (k % E == 0 && n % E == 0 && opl::aligned16(a) && opl::aligned16(b)) return kAligned16;
  const bool dword_rows = k * sizeof(T) % 4 == 0 && n * sizeof(T) % 4 == 0 &&
                          reinterpret_cast<std::uintptr_t>(a) % 4 == 0 &&
                          reinterpret_cast<std::uintptr_t>(b) % 4 == 0;
  return dword_rows ? kDword : kElementwise;
}

int device_cus();

template <typename Cfg>
hipError_t launch_dma_tiles(const typename Cfg::Type* a, const typename Cfg::Type* b, float* c,
                            int m, int n, int k, int lda, int ldb, hipStream_t stream,
                            dma::TailSplit tail = {0, 0, 0, nullptr}) {
  const long long tiles = static_cast<long long>((m + Cfg::kBM - 1) / Cfg::kBM) *
                          ((n + Cfg::kBN - 1) / Cfg::kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const long long blocks =
      tail.splits > 0 ? tail.full_tiles + static_cast<long long>(tail.tiles) * tail.splits : tiles;
  // Shapes with a partly filled last K step, or fp16 rows of odd length,
  // run the instance that repairs that step (the others keep the plain
  // schedule: the repair's code cost the aligned 4096^3 product 2%).
  const bool edge = k % Cfg::kBK != 0 || (sizeof(typename Cfg::Type) == 2 && (lda % 2 != 0 || ldb % 2 != 0));
  // C is stored non-temporally when later rounds re-read operand panels
  // that cached C lines would evict: fp16 256 x 256 grids (whose whole
  // tiles leave through LDS as full cache lines) of two or more rounds,
  // with A and B together past three quarters of the 256 MiB Infinity
  // Cache. Measured on MI355X (us, cached -> non-temporal, both with the
  // staged epilogue): 8192^3 (A + B 256 MiB) 852 -> 770; 16384^2 x 4096
  // (256 MiB) 1811 -> 1604; 12288^2 x 8192 (384 MiB) 1945 -> 1741;
  // 8192^2 x 4096 (128 MiB) 405.5 -> 404.9; 8192^2 x 2048 (64 MiB) 226.6
  // -> 230.2; 4096 x 8192 x 4096 (96 MiB) 202.4 -> 207.0; single rounds
  // lose (4096^3 104.0 -> 108.2, 4095^3 128 -> 166). Rows at any 4-byte
  // phase stream too: 8191^3 948 -> 920 with the staged stores (the
  // per-float stores had lost there, 948 -> 1063).
  constexpr bool kCanStream =
      sizeof(typename Cfg::Type) == 2 && Cfg::kBM == 256 && Cfg::kStages == 2;
  const long long operand_bytes =
      (static_cast<long long>(m) * lda + static_cast<long long>(k) * ldb) *
      static_cast<long long>(sizeof(typename Cfg::Type));
  const bool stream_c = kCanStream && tail.splits == 0 && operand_bytes >= (192LL << 20) &&
                        device_cus() > 0 && tiles >= 2LL * device_cus();
  const dim3 grid(static_cast<unsigned>(blocks)), block(Cfg::kThreads);
  if (tail.splits > 0) {
    if (edge)
      dma::gemm_dma_kernel<Cfg, true, true><<<grid, block, 0, stream>>>(a, b, c, m, n, k, lda,
                                                                        ldb, tail);
    else
      dma::gemm_dma_kernel<Cfg, true><<<grid, block, 0, stream>>>(a, b, c, m, n, k, lda, ldb,
                                                                  tail);
    dma::sum_tail_kernel<Cfg><<<dim3(Cfg::kBM * Cfg::kBN / 4 / 256, tail.tiles), dim3(256), 0,
                                stream>>>(c, m, n, tail);
  } else if (stream_c) {
    if constexpr (kCanStream) {
      if (edge)
        dma::gemm_dma_kernel<Cfg, false, true, true><<<grid, block, 0, stream>>>(
            a, b, c, m, n, k, lda, ldb, tail);
      else
        dma::gemm_dma_kernel<Cfg, false, false, true><<<grid, block, 0, stream>>>(
            a, b, c, m, n, k, lda, ldb, tail);
    }
  } else if (edge) {
    dma::gemm_dma_kernel<Cfg, false, true><<<grid, block, 0, stream>>>(a, b, c, m, n, k, lda,
                                                                       ldb, tail);
  } else {
    dma::gemm_dma_kernel<Cfg><<<grid, block, 0, stream>>>(a, b, c, m, n, k, lda, ldb, tail);
  }
  return hipGetLastError();
}

// A 256 x 256-tile grid that fills R >= 1 rounds of one workgroup per CU
// plus a last round at most half full leaves most CUs idle for a whole
// tile's time: the last round's tiles are then split along K into enough
// parts to fill the CUs (at most 16, at least 256 deep each, and as many as
// their partial tiles fit the call's scratch) and summed by a second
// launch. Measured on MI355X (us, unsplit vs split): 4096 x 4160 x 4096 (272
// tiles, 16 in the last round: 16 parts of 4 K steps) 180-185 vs 138-143;
// 4160 x 4096 x 4032 (15 uneven parts) 184 vs 145; 4100 x 4104 x 2048 (289
// tiles, 33 last: 7 parts) 101 vs 93. Last rounds more than half full stay
// unsplit (4096 x 11008: 688 tiles, 176 last).
constexpr int kTailMaxSplits = 16;
constexpr int kTailMinDepth = 256;

// CUs of the current device, looked up once per device (0 if unknown).
int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> known[kMaxDevices] = {};
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 0;
  if (device >= 0 && device < kMaxDevices) {
    const int cached = known[device].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  if (device >= 0 && device < kMaxDevices) known[device].store(cus, std::memory_order_relaxed);
  return cus;
}

// Grids of fewer 256 x 256 tiles than this run on 128 x 128 tiles. Measured
// on MI355X (us, 256 x 256 vs 128 x 128 tiles): 1000 x 4096 x 4096 (64
// tiles) 85.9 vs 45.9; 2048 x 4096 x 4096 (128) 89.1 vs 69.7; 2304 x 5120 x
// 4096 (180) 102.8 vs 110.0; 4096^3 (256) 121.1 vs 136.5.
constexpr long long kSmallGridTiles = 160;

// The direct-to-LDS tile configurations of an element type, and the grid
// (in 256 x 256 tiles) below which the 128 x 128 ones run.
template <typename T>
struct DmaTiles;
template <>
struct DmaTiles<_Float16> {
  using Big = dma::BigTile;
  using BigHalfK = dma::BigTileK32;  // K % 64 == 32
  using Small = dma::SmallTile;
  static constexpr long long kSmallBelow = kSmallGridTiles;
};
template <>
struct DmaTiles<float> {
  using Big = dma::BigTileF32;
  using BigHalfK = dma::BigTileF32K16;  // K % 32 == 16
  using Small = dma::SmallTileF32;
  static constexpr long long kSmallBelow = kSmallGridTilesF32;
};

// Split of the last round of a 256 x 256-tile grid (splits == 0: none).
struct TailPlan {
  int splits = 0;
  long long full = 0;  // tiles computed whole, before the split ones
  long long last = 0;  // tiles split along K (the last round, or all)
  std::size_t bytes = 0;
};

// Grids of 128 x 128 tiles (two workgroups per CU) with fewer tiles than
// CUs split every tile along K instead, into as many parts as fill the
// workgroup slots (same limits). Small M past the skinny kernels' 16 rows
// is the case: M = 17..128, N = K = 4096 is 32 tiles. Measured on MI355X
// (us, whole tiles -> split, B cycling through 8 copies):
//   fp16 M = 17 30.4 -> 19.7, M = 64 31.8 -> 23.1, M = 128 37.1 -> 29.5,
//     M = 256 39.4 -> 32.7;
//   fp32 M = 17 236.8 -> 43.4, M = 64 238.3 -> 46.1, M = 128 237.9 ->
//     48.0, M = 256 239.4 -> 75.6.
template <typename T>
TailPlan tail_plan(int m, int n, int k, std::size_t capacity) {
  TailPlan t;
  const int cus = device_cus();
  if (cus <= 0) return t;
  const long long big_tiles =
      static_cast<long long>((m + dma::BigTile::kBM - 1) / dma::BigTile::kBM) *
      ((n + dma::BigTile::kBN - 1) / dma::BigTile::kBN);
  long long split_tiles = 0, full = 0, want = 0;
  std::size_t tile_bytes = 0;
  if (big_tiles < DmaTiles<T>::kSmallBelow) {
    using Small = typename DmaTiles<T>::Small;
    const long long tiles = static_cast<long long>((m + Small::kBM - 1) / Small::kBM) *
                            ((n + Small::kBN - 1) / Small::kBN);
    if (tiles >= cus) return t;
    split_tiles = tiles;
    want = 2LL * cus / tiles;
    tile_bytes = static_cast<std::size_t>(Small::kBM) * Small::kBN * sizeof(float);
  } else {
    const long long last = big_tiles % cus;
    if (big_tiles <= cus || last == 0 || last > cus / 2) return t;
    split_tiles = last;
    full = big_tiles - last;
    want = cus / last;
    tile_bytes = static_cast<std::size_t>(dma::BigTile::kBM) * dma::BigTile::kBN * sizeof(float);
  }
  const std::size_t per_split = static_cast<std::size_t>(split_tiles) * tile_bytes;
  long long splits = want;
  if (splits > kTailMaxSplits) splits = kTailMaxSplits;
  if (splits > k / kTailMinDepth) splits = k / kTailMinDepth;
  if (static_cast<std::size_t>(splits) > capacity / per_split)
    splits = static_cast<long long>(capacity / per_split);
  if (splits < 2) return t;
  t.splits = static_cast<int>(splits);
  t.full = full;
  t.last = split_tiles;
  t.bytes = per_split * static_cast<std::size_t>(splits);
  return t;
}

// The direct-to-LDS kernel (any K, N and alignment) on 128 x 128 or 256 x 256
// tiles, with `tail` split into `partials` (tail.bytes of scratch).
template <typename T>
hipError_t launch_gemm_dma(const T* a, const T* b, float* c, int m, int n, int k, int lda, int ldb,
                           const TailPlan& tail, void* partials, hipStream_t stream) {
  using Tiles = DmaTiles<T>;
  static_assert(Tiles::Big::kBM == dma::BigTile::kBM && Tiles::Big::kBN == dma::BigTile::kBN &&
                    Tiles::BigHalfK::kBM == dma::BigTile::kBM &&
                    Tiles::BigHalfK::kBN == dma::BigTile::kBN,
                "one big tile size");
  const long long big_tiles =
      static_cast<long long>((m + dma::BigTile::kBM - 1) / dma::BigTile::kBM) *
      ((n + dma::BigTile::kBN - 1) / dma::BigTile::kBN);
  dma::TailSplit split{0, 0, 0, nullptr};
  if (tail.splits > 0)
    split = dma::TailSplit{static_cast<int>(tail.full), static_cast<int>(tail.last), tail.splits,
                           static_cast<float*>(partials)};
  if (big_tiles < Tiles::kSmallBelow)
    return launch_dma_tiles<typename Tiles::Small>(a, b, c, m, n, k, lda, ldb, stream, split);
  // A last step at most half full runs on the half-deep stages.
  const int rest = k % Tiles::Big::kBK;
  if (rest == 0 || rest > Tiles::BigHalfK::kBK)
    return launch_dma_tiles<typename Tiles::Big>(a, b, c, m, n, k, lda, ldb, stream, split);
  return launch_dma_tiles<typename Tiles::BigHalfK>(a, b, c, m, n, k, lda, ldb, stream, split);
}

// One call's plan and the scratch it needs.
struct GemmPlan {
  enum Kind { kSkinny, kNarrow, kDma, kRegister } kind = kRegister;
  skinny::Plan skinny;
  TailPlan tail;  // kDma
  PadPlan pad;    // kDma
  int staging = kElementwise;  // kRegister
  std::size_t bytes = 0;
};

template <typename T>
GemmPlan plan_gemm(const T* a, const T* b, int m, int n, int k, std::size_t capacity) {
  GemmPlan p;
  if (skinny::applies(b, m, n)) {
    p.skinny = skinny::plan<T>(m, n, k, capacity);
    if (p.skinny.ok) {
      p.kind = GemmPlan::kSkinny;
      p.bytes = p.skinny.bytes;
      return p;
    }
  }
  if (narrow::applies(a, b, n, k)) {
    p.kind = GemmPlan::kNarrow;
    return p;
  }
  // The copy kernel's per-lane offsets inside a tile are 32-bit: up to
  // 255 rows of A (255 * K * sizeof(T) bytes) and one K step of B rows (64
  // fp16 or 32 fp32 rows: 128 * N bytes).
  const bool dma_offsets_fit = k < (sizeof(T) == 2 ? (1 << 22) : (1 << 21)) && n < (1 << 24);
  if (dma_offsets_fit) {
    p.kind = GemmPlan::kDma;
    p.pad = pad_plan<T>(a, b, m, n, k);
    if (p.pad.bytes() > capacity) p.pad = PadPlan{false, false, k, k, n, 0, 0};
    // The split partials of a partly filled last round follow the copies,
    // in what is left of the capacity.
    p.tail = tail_plan<T>(m, n, p.pad.k, capacity - p.pad.bytes());
    p.bytes = p.pad.bytes() + p.tail.bytes;
    return p;
  }
  p.kind = GemmPlan::kRegister;
  p.staging = staging_for<T>(a, b, n, k);
  return p;
}

// Runs plan `p`; `scratch` holds p.bytes (unused when 0).
template <typename T>
hipError_t run_gemm(const GemmPlan& p, const T* a, const T* b, float* c, int m, int n, int k,
                    opl::ScratchLease* lease, hipStream_t stream) {
  void* const scratch = lease != nullptr ? lease->data() : nullptr;
  switch (p.kind) {
    case GemmPlan::kSkinny:
      return skinny::launch<T>(a, b, c, m, n, k, p.skinny, scratch, lease, stream);
    case GemmPlan::kNarrow:
      return narrow::launch<T>(a, b, c, m, n, k, stream);
    case GemmPlan::kDma: {
      const T* pa = a;
      const T* pb = b;
      unsigned char* const ws = static_cast<unsigned char*>(scratch);
      if constexpr (sizeof(T) == 2) {
        // Both copies' sizes are rounded to 256 bytes: the partials start aligned.
        if (p.pad.pad_a) {
          launch_pad_copy(a, m, k, reinterpret_cast<T*>(ws), m, p.pad.lda, stream);
          pa = reinterpret_cast<const T*>(ws);
        }
        if (p.pad.pad_b) {
          launch_pad_copy(b, k, n, reinterpret_cast<T*>(ws + p.pad.a_bytes), p.pad.k,
                          p.pad.ldb, stream);
          pb = reinterpret_cast<const T*>(ws + p.pad.a_bytes);
        }
      }
      void* const partials = ws != nullptr ? ws + p.pad.bytes() : nullptr;
      return launch_gemm_dma<T>(pa, pb, c, m, n, p.pad.k, p.pad.lda, p.pad.ldb, p.tail,
                                partials, stream);
    }
    default:
      return launch_generic_for<T>(p.staging, a, b, c, m, n, k, n, stream);
  }
}

// A GEMM call with its scratch from `src`; query != nullptr only reports the
// plan's scratch bytes (nothing is enqueued).
template <typename T>
int gemm_entry(const T* a, const T* b, float* c, int m, int n, int k,
               const opl::ScratchSource& src, std::size_t* query, hipStream_t stream) {
  const GemmPlan p = plan_gemm<T>(a, b, m, n, k, src.capacity());
  if (query != nullptr) {
    *query = p.bytes;
    return hipSuccess;
  }
  if (src.workspace_mode && !opl::workspace_ok(src.data, src.bytes, p.bytes))
    return hipErrorInvalidValue;
  if (p.bytes == 0) return run_gemm<T>(p, a, b, c, m, n, k, nullptr, stream);
  // Held until the last kernel that reads the scratch is enqueued.
  opl::ScratchLease lease(stream, src.workspace_mode ? src.data : nullptr, src.bytes);
  if (lease.status() != hipSuccess) return lease.status();
  return run_gemm<T>(p, a, b, c, m, n, k, &lease, stream);
}

const _Float16* as_f16(const operatorlib_half_t* p) {
  return reinterpret_cast<const _Float16*>(p);
}

}  // namespace

extern "C" int operatorlib_gemm_f32(const float* a, const float* b, float* c,
                                    int m, int n, int k,
                                    void* stream_handle) {
  if (!opl::gemm_args_ok(a, b, c, m, n, k)) return hipErrorInvalidValue;
  return gemm_entry<float>(a, b, c, m, n, k, opl::ScratchSource{}, nullptr,
                           static_cast<hipStream_t>(stream_handle));
}

extern "C" int operatorlib_gemm_f16(const operatorlib_half_t* a,
                                    const operatorlib_half_t* b, float* c,
                                    int m, int n, int k,
                                    void* stream_handle) {
  if (!opl::gemm_args_ok(a, b, c, m, n, k)) return hipErrorInvalidValue;
  return gemm_entry<_Float16>(as_f16(a), as_f16(b), c, m, n, k, opl::ScratchSource{}, nullptr,
                              static_cast<hipStream_t>(stream_handle));
}

extern "C" size_t operatorlib_gemm_f32_workspace_size(const float* a, const float* b, int m,
                                                      int n, int k) {
  if (!opl::gemm_args_ok(a, b, a, m, n, k)) return 0;
  std::size_t bytes = 0;
  gemm_entry<float>(a, b, nullptr, m, n, k, opl::ScratchSource{true, nullptr, 0}, &bytes,
                    nullptr);
  return bytes;
}

extern "C" size_t operatorlib_gemm_f16_workspace_size(const operatorlib_half_t* a,
                                                      const operatorlib_half_t* b, int m,
                                                      int n, int k) {
  if (!opl::gemm_args_ok(a, b, a, m, n, k)) return 0;
  std::size_t bytes = 0;
  gemm_entry<_Float16>(as_f16(a), as_f16(b), nullptr, m, n, k,
                       opl::ScratchSource{true, nullptr, 0}, &bytes, nullptr);
  return bytes;
}

extern "C" int operatorlib_gemm_f32_ws(const float* a, const float* b, float* c, int m, int n,
                                       int k, void* workspace, size_t workspace_bytes,
                                       void* stream_handle) {
  if (!opl::gemm_args_ok(a, b, c, m, n, k)) return hipErrorInvalidValue;
  return gemm_entry<float>(a, b, c, m, n, k,
                           opl::ScratchSource{true, workspace, workspace_bytes}, nullptr,
                           static_cast<hipStream_t>(stream_handle));
}

extern "C" int operatorlib_gemm_f16_ws(const operatorlib_half_t* a, const operatorlib_half_t* b,
                                       float* c, int m, int n, int k, void* workspace,
                                       size_t workspace_bytes, void* stream_handle) {
  if (!opl::gemm_args_ok(a, b, c, m, n, k)) return hipErrorInvalidValue;
  return gemm_entry<_Float16>(as_f16(a), as_f16(b), c, m, n, k,
                              opl::ScratchSource{true, workspace, workspace_bytes}, nullptr,
                              static_cast<hipStream_t>(stream_handle));
}
