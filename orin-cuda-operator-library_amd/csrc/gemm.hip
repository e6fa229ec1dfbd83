// Row-major GEMM C[M,N] = A[M,K] * B[K,N] on the CDNA4 matrix cores.
//   gemm_f16: fp16 A/B, v_mfma_f32_32x32x16_f16, fp32 accumulate and output
//   gemm_f32: fp32 A/B, v_mfma_f32_32x32x2_f32,  fp32 accumulate and output
//
// Reference: operatorlib::gemm_f16 / gemm_f32 (src/gemm.cu:440-479). The
// reference dispatches between WMMA, cp.async register-tiled and scalar
// kernels on divisibility; here one MFMA kernel template serves every shape:
// the "vector" instance stages 16-byte chunks and needs 16-byte aligned
// rows, the "general" instance stages element by element with zero fill and
// takes any shape and alignment (the 4095^3 edge case runs on MFMA too).
//
// Tiling (both precisions):
//   * 256 x 256 C tile per 256-thread workgroup; 2 x 2 wavefronts, each
//     owning a 128 x 128 sub-tile = 4 x 4 MFMA 32x32 blocks (256 fp32
//     accumulators per lane, held in AGPR/VGPR at one wave per SIMD);
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

#include <cstddef>
#include <cstdint>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "validate.hpp"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kWaveM = 128;
constexpr int kWaveN = 128;
constexpr int kFragsM = kWaveM / 32;  // 4
constexpr int kFragsN = kWaveN / 32;  // 4
constexpr int kRowBytes = 128;        // one K step of one row
constexpr int kChunksPerRow = kRowBytes / 16;
constexpr int kPitch = kRowBytes + 16;  // padded LDS row
constexpr int kTileABytes = kBM * kPitch;
constexpr int kTileBBytes = kBN * kPitch;
constexpr int kStageBytes = kTileABytes + kTileBBytes;
constexpr int kLdsBytes = 2 * kStageBytes;  // 147456 of 163840
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

template <typename T, bool kVector>
struct Stager {
  using P = Precision<T>;
  using Chunk = typename P::Chunk;
  static constexpr int E = P::kChunkElems;
  static constexpr int kBK = kRowBytes / sizeof(T);  // K elements per step
  // A: kBM rows x kChunksPerRow chunks; each thread stages kAChunks.
  static constexpr int kAChunks = kBM * kChunksPerRow / kThreads;  // 8
  // B: E x E element blocks (E k-rows x one n-chunk); kBBlocks per thread.
  static constexpr int kBBlocks =
      (kBK / E) * (kBN / E) / kThreads;  // fp16: 1, fp32: 2

  Chunk a[kAChunks];
  Chunk b[kBBlocks][E];

  __device__ __forceinline__ static Chunk load_chunk(const T* base,
                                                     std::size_t ld, int row,
                                                     int rows, int col,
                                                     int cols) {
    Chunk v;
    if constexpr (kVector) {
      // Vector instances need cols % E == 0, so a chunk is all in or out.
      if (row < rows && col < cols) {
        v = *reinterpret_cast<const Chunk*>(
            base + static_cast<std::size_t>(row) * ld + col);
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = T(0);
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
  __device__ __forceinline__ void load(const T* A, const T* B, int M, int N,
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
        b[blk][r] = load_chunk(B, N, k0 + g * E + r, K, n0 + j * E, N);
    }
  }

  // Registers -> LDS stage (A as [m][k], B transposed to [n][k]).
  __device__ __forceinline__ void store(unsigned char* stage) const {
    const int tid = threadIdx.x;
    unsigned char* sa = stage;
    unsigned char* sb = stage + kTileABytes;
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

// Maps the launch index to a C tile: first regroups the round-robin XCD
// dispatch so consecutive tiles land on one XCD, then walks tiles in
// column-major groups of kGroupM tile-rows.
__device__ __forceinline__ void tile_of_block(int tiles_m, int tiles_n,
                                              int* tm, int* tn) {
  const int blocks = gridDim.x;
  int bid = blockIdx.x;
  if (blocks % kXcds == 0)
    bid = (bid % kXcds) * (blocks / kXcds) + bid / kXcds;
  const int group_size = kGroupM * tiles_n;
  const int first_m = (bid / group_size) * kGroupM;
  const int rows_in_group = min(tiles_m - first_m, kGroupM);
  const int in_group = bid % group_size;
  *tm = first_m + in_group % rows_in_group;
  *tn = in_group / rows_in_group;
}

template <typename T, bool kVector>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_mfma_kernel(const T* __restrict__ A, const T* __restrict__ B,
                      float* __restrict__ C, int M, int N, int K) {
  using P = Precision<T>;
  using Chunk = typename P::Chunk;
  using S = Stager<T, kVector>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];

  const int tiles_m = (M + kBM - 1) / kBM;
  const int tiles_n = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_of_block(tiles_m, tiles_n, &tm, &tn);
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;

  const int lane = threadIdx.x % opl::kWaveSize;
  const int wave = threadIdx.x / opl::kWaveSize;
  const int wm = wave / 2;
  const int wn = wave % 2;
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
  stager.load(A, B, M, N, K, m0, n0, 0);
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
      stager.load(A, B, M, N, K, m0, n0, (step + 1) * S::kBK);
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

template <typename T>
hipError_t launch_gemm(const T* a, const T* b, float* c, int m, int n, int k,
                       hipStream_t stream) {
  constexpr int E = Precision<T>::kChunkElems;
  const bool vector_ok = k % E == 0 && n % E == 0 && opl::aligned16(a) &&
                         opl::aligned16(b);
  const long long tiles = static_cast<long long>((m + kBM - 1) / kBM) *
                          ((n + kBN - 1) / kBN);
  if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(tiles)), block(kThreads);
  if (vector_ok)
    gemm_mfma_kernel<T, true><<<grid, block, 0, stream>>>(a, b, c, m, n, k);
  else
    gemm_mfma_kernel<T, false><<<grid, block, 0, stream>>>(a, b, c, m, n, k);
  return hipGetLastError();
}

}  // namespace

extern "C" int operatorlib_gemm_f32(const float* a, const float* b, float* c,
                                    int m, int n, int k,
                                    void* stream_handle) {
  if (!opl::gemm_args_ok(a, b, c, m, n, k)) return hipErrorInvalidValue;
  return launch_gemm<float>(a, b, c, m, n, k,
                            static_cast<hipStream_t>(stream_handle));
}

extern "C" int operatorlib_gemm_f16(const operatorlib_half_t* a,
                                    const operatorlib_half_t* b, float* c,
                                    int m, int n, int k,
                                    void* stream_handle) {
  if (!opl::gemm_args_ok(a, b, c, m, n, k)) return hipErrorInvalidValue;
  return launch_gemm<_Float16>(reinterpret_cast<const _Float16*>(a),
                               reinterpret_cast<const _Float16*>(b), c, m, n,
                               k, static_cast<hipStream_t>(stream_handle));
}
