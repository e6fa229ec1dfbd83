// softmax_f32 / softmax_f16: numerically stable softmax over the last
// dimension of a row-major [rows, cols] matrix; fp16 rows are computed in
// fp32 and rounded to fp16 once, on store.
//
// Reference: operatorlib::softmax_f32 (src/softmax.cu:182-202) with three
// CUDA kernels (:52-176); its general path reads the input twice and the
// output twice. Same maths here:
//   m = max_c x[c];  p[c] = exp(x[c] - m);  out[c] = p[c] * (1 / sum_c p[c])
// with exp evaluated as exp2((x - m) * log2 e) on v_exp_f32. The fp16
// variant is the "FP16 input, FP32 accumulation" extension the reference
// defers (softmax/reports/v4.md:140-141, docs/pytorch_extension.md:143-146).
//
// MI355X design: the row stays in VGPRs between the max, exp/sum and scale
// steps, so every path up to 32768 columns reads x once and writes once
// (the HBM minimum: 8 bytes per fp32 element, 4 per fp16). Reductions are
// wave64 DPP butterflies (plus an 8-slot LDS combine for workgroup rows).
// Rows longer than 32768 columns use an online (max, sum) first pass and
// re-read x once.
// Padding slots hold -inf, which exp maps to 0.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "rowwise.hpp"
#include "validate.hpp"

namespace {

using opl::kLog2e;

template <int N>
__device__ __forceinline__ float local_max(const float (&x)[N]) {
  float m = x[0];
#pragma unroll
  for (int i = 1; i < N; ++i) m = fmaxf(m, x[i]);
  return m;
}

// exp(x - m) in place; returns the thread's sum of the new values.
template <int N>
__device__ __forceinline__ float exp_shift_sum(float (&x)[N], float m) {
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    x[i] = opl::fast_exp2((x[i] - m) * kLog2e);
    sum += x[i];
  }
  return sum;
}

template <int N>
__device__ __forceinline__ void scale(float (&x)[N], float s) {
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] *= s;
}

template <typename T, int V, int W>
__global__ __launch_bounds__(opl::kRowWaveThreads) void softmax_wave_kernel(
    const T* __restrict__ input, T* __restrict__ output, int rows, int cols) {
  const int lane = threadIdx.x % opl::kWaveSize;
  const int row = blockIdx.x * opl::kRowWaveRows + threadIdx.x / opl::kWaveSize;
  if (row >= rows) return;  // uniform per wavefront
  const std::size_t offset = static_cast<std::size_t>(row) * cols;
  typename opl::SliceFor<V, opl::kWaveSize, W, T>::type s;
  s.template load<true>(input + offset, cols, lane, -INFINITY);
  const float m = opl::wave_reduce<opl::MaxOp>(local_max(s.x));
  const float sum = opl::wave_reduce<opl::SumOp>(exp_shift_sum(s.x, m));
  scale(s.x, 1.0f / sum);
  s.store(output + offset, cols, lane);
}

template <typename T, int V, int W>
__global__ __launch_bounds__(opl::kRowBlockThreads) void softmax_block_kernel(
    const T* __restrict__ input, T* __restrict__ output, int cols) {
  __shared__ float max_slots[opl::kRowBlockWaves];
  __shared__ float sum_slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  typename opl::SliceFor<V, opl::kRowBlockThreads, W, T>::type s;
  s.template load<true>(input + offset, cols, threadIdx.x, -INFINITY);
  const float m = opl::block_reduce<opl::MaxOp, opl::kRowBlockWaves>(
      local_max(s.x), max_slots);
  const float sum = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(
      exp_shift_sum(s.x, m), sum_slots);
  scale(s.x, 1.0f / sum);
  s.store(output + offset, cols, threadIdx.x);
}

// Online (running max, rescaled running sum) update for one element.
__device__ __forceinline__ void online_update(float x, float& m, float& s) {
  if (x > m) {
    s = s * opl::fast_exp2((m - x) * kLog2e) + 1.0f;
    m = x;
  } else {
    s += opl::fast_exp2((x - m) * kLog2e);
  }
}

// Rows longer than the register slices: pass 1 keeps an online (max, sum)
// per thread, pass 2 re-reads the row and writes exp(x - max) / sum.
// `vec` selects 16-byte chunk accesses (cols % E == 0, aligned rows).
template <typename T>
__global__ __launch_bounds__(opl::kRowBlockThreads) void softmax_two_pass_kernel(
    const T* __restrict__ input, T* __restrict__ output, int cols, int vec) {
  using Chunk = typename opl::RowElem<T>::Chunk;
  constexpr int E = opl::RowElem<T>::kPerChunk;
  __shared__ float max_slots[opl::kRowBlockWaves];
  __shared__ float sum_slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  const T* row = input + offset;
  T* out = output + offset;
  const int t = threadIdx.x;
  constexpr int kT = opl::kRowBlockThreads;
  float m = -FLT_MAX;
  float s = 0.0f;
  if (vec) {
    const Chunk* rc = reinterpret_cast<const Chunk*>(row);
    for (int i = t; i < cols / E; i += kT) {
      const Chunk q = rc[i];
#pragma unroll
      for (int e = 0; e < E; ++e) online_update(static_cast<float>(q[e]), m, s);
    }
  } else {
    for (int c = t; c < cols; c += kT)
      online_update(static_cast<float>(row[c]), m, s);
  }
  const float row_max =
      opl::block_reduce<opl::MaxOp, opl::kRowBlockWaves>(m, max_slots);
  const float row_sum = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(
      s * opl::fast_exp2((m - row_max) * kLog2e), sum_slots);
  const float inv = 1.0f / row_sum;
  if (vec) {
    const Chunk* rc = reinterpret_cast<const Chunk*>(row);
    Chunk* oc = reinterpret_cast<Chunk*>(out);
    for (int i = t; i < cols / E; i += kT) {
      const Chunk q = rc[i];
      Chunk y;
#pragma unroll
      for (int e = 0; e < E; ++e)
        y[e] = static_cast<T>(
            opl::fast_exp2((static_cast<float>(q[e]) - row_max) * kLog2e) * inv);
      oc[i] = y;
    }
  } else {
    for (int c = t; c < cols; c += kT)
      out[c] = static_cast<T>(
          opl::fast_exp2((static_cast<float>(row[c]) - row_max) * kLog2e) * inv);
  }
}

// Ragged fp32 rows of up to kTileMaxCols columns (cols % 4 != 0 or
// unaligned rows) as flat tiles: a workgroup's 4 consecutive rows are one
// contiguous range of the matrix, moved between HBM and LDS in aligned
// 16-byte chunks (scalar accesses only for the range's first and last
// partial chunk), and each wavefront reduces its row out of LDS. Per-row
// misaligned starts cost the one-row-per-wavefront kernel ~1 us per 4097 x
// 1023 call (7.6 us against 6.0 aligned); here only every fourth row
// boundary is a chunk boundary shared with another workgroup. Measured on
// MI355X (us, cold buffers): 4097 x 1023 7.62 -> 7.06, 8191 x 511 7.99 ->
// 7.69. 8 rows per workgroup: 7.13 / 6.92; 16: 8.23 / 6.75. fp16 rows and
// longer rows measured slower this way (4097 x 1023 fp16 4.78 -> 5.64,
// 2047 x 4095 12.90 -> 13.39: the fp32 tile doubles the fp16 bytes through
// LDS, and 64 KiB tiles halve the workgroups per CU), so they keep the
// wavefront kernel. V: columns per lane / 4.
constexpr int kTileMaxCols = 1024;
template <int V>
__global__ __launch_bounds__(opl::kRowWaveThreads) void softmax_tile_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows, int cols) {
  typedef float F4 __attribute__((ext_vector_type(4)));
  constexpr int kT = opl::kRowWaveThreads;
  constexpr int kRows = opl::kRowWaveRows;
  constexpr int kPerLane = 4 * V;  // row elements per lane
  // kRows rows of up to 64 * kPerLane columns, plus one chunk of lead-in
  __shared__ __attribute__((aligned(16))) float tile[kRows * opl::kWaveSize * kPerLane + 4];
  const int t = threadIdx.x;
  const int r0 = blockIdx.x * kRows;
  const int nrows = min(kRows, rows - r0);
  const int n = nrows * cols;  // elements of the range, >= 8
  const float* in = input + static_cast<std::size_t>(r0) * cols;
  float* out = output + static_cast<std::size_t>(r0) * cols;
  // Range element k sits at tile[lead + k]: lead is the range start's
  // offset from the 16-byte boundary below it, so every aligned chunk of the
  // range is an aligned 16-byte LDS slot too (output rows share the input's
  // phase, so the same chunks are aligned there).
  const int lead = static_cast<int>((reinterpret_cast<uintptr_t>(in) & 15) / 4);
  const int head = (4 - lead) % 4;  // elements before the first boundary
  const int body = (n - head) / 4;  // aligned chunks, >= 1
  const int tail0 = head + 4 * body;
  // Thread t loads chunks t + kT * j (indices clamped: loads issue back to
  // back, out-of-range ones are dropped on the LDS write); threads 0 .. head-1
  // take the head elements, threads 4 .. 4 + (n - tail0) - 1 the tail.
  const F4* bin = reinterpret_cast<const F4*>(in + head);
  F4 q[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = t + kT * j;
    q[j] = __builtin_nontemporal_load(bin + (c < body ? c : 0));
  }
  const int xc = t < head ? t : (t >= 4 && t - 4 < n - tail0 ? tail0 + t - 4 : -1);
  const float xv = in[xc >= 0 ? xc : 0];
  float* const base = tile + lead + head;  // 16-byte aligned
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = t + kT * j;
    if (c < body) *reinterpret_cast<F4*>(base + 4 * c) = q[j];
  }
  if (xc >= 0) tile[lead + xc] = xv;
  __syncthreads();
  const int w = t / opl::kWaveSize;
  const int lane = t % opl::kWaveSize;
  if (w < nrows) {
    float* const rowp = tile + lead + w * cols;
    float x[kPerLane];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const int c = lane + opl::kWaveSize * i;
      x[i] = c < cols ? rowp[c] : -INFINITY;
    }
    const float m = opl::wave_reduce<opl::MaxOp>(local_max(x));
    const float sum = opl::wave_reduce<opl::SumOp>(exp_shift_sum(x, m));
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const int c = lane + opl::kWaveSize * i;
      if (c < cols) rowp[c] = x[i] * inv;
    }
  }
  __syncthreads();
  F4* const bout = reinterpret_cast<F4*>(out + head);
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = t + kT * j;
    if (c < body)
      __builtin_nontemporal_store(*reinterpret_cast<const F4*>(base + 4 * c), bout + c);
  }
  if (xc >= 0) __builtin_nontemporal_store(tile[lead + xc], out + xc);
}

template <int V>
void launch_tile(int v, const float* in, float* out, int rows, int cols,
                 hipStream_t stream) {
  if constexpr (4 * V * opl::kWaveSize < kTileMaxCols) {
    if (v > V) return launch_tile<2 * V>(v, in, out, rows, cols, stream);
  }
  const int blocks = (rows + opl::kRowWaveRows - 1) / opl::kRowWaveRows;
  softmax_tile_kernel<V><<<dim3(blocks), dim3(opl::kRowWaveThreads), 0, stream>>>(
      in, out, rows, cols);
}

// Launches the kernel instance whose per-thread count V is the smallest power
// of two >= v (v comes from pick_row_plan, so it never exceeds MaxV).
template <typename T, int W, int V, int MaxV>
void launch_wave(int v, const T* in, T* out, int rows, int cols,
                 hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V)
      return launch_wave<T, W, 2 * V, MaxV>(v, in, out, rows, cols, stream);
  }
  const int blocks = (rows + opl::kRowWaveRows - 1) / opl::kRowWaveRows;
  softmax_wave_kernel<T, V, W><<<dim3(blocks), dim3(opl::kRowWaveThreads), 0,
                                 stream>>>(in, out, rows, cols);
}

template <typename T, int W, int V, int MaxV>
void launch_block(int v, const T* in, T* out, int rows, int cols,
                  hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V)
      return launch_block<T, W, 2 * V, MaxV>(v, in, out, rows, cols, stream);
  }
  softmax_block_kernel<T, V, W><<<dim3(rows), dim3(opl::kRowBlockThreads),
                                  0, stream>>>(in, out, cols);
}

// Shared dispatch of the fp32 and fp16 entry points. E elements per 16-byte
// chunk; per-thread counts V run from the smallest a path can see up to the
// register budget (64 fp32 values per thread).
template <typename T>
int softmax_launch(const T* input, T* output, int rows, int cols,
                   hipStream_t stream) {
  constexpr int E = opl::RowElem<T>::kPerChunk;
  constexpr int kWaveMaxV = opl::kRowWaveMaxCols / (opl::kWaveSize * E);
  constexpr int kBlockMinV =
      2 * opl::kRowWaveMaxCols / (opl::kRowBlockThreads * E);
  constexpr int kBlockMaxV =
      opl::kRowBlockMaxCols / (opl::kRowBlockThreads * E);
  const bool vec =
      cols % E == 0 && opl::aligned16(input) && opl::aligned16(output);
  // Ragged rows (cols % E != 0 or unaligned) keep 16-byte accesses when
  // input and output rows share their 16-byte phase.
  const bool ragged =
      !vec && opl::same_phase16(input, output) &&
      cols >= opl::RaggedRowSlice<1, opl::kWaveSize, T>::kMinCols;
  const opl::RowPlan plan = opl::pick_row_plan(cols, vec || ragged ? E : 1);
  switch (plan.path) {
    case opl::RowPath::kWave:
      if (vec) launch_wave<T, E, 1, kWaveMaxV>(plan.per_thread, input, output, rows, cols, stream);
      else if (ragged && std::is_same<T, float>::value && cols <= kTileMaxCols)
        launch_tile<1>(plan.per_thread, reinterpret_cast<const float*>(input),
                       reinterpret_cast<float*>(output), rows, cols, stream);
      else if (ragged) launch_wave<T, 0, 1, kWaveMaxV>(plan.per_thread, input, output, rows, cols, stream);
      else launch_wave<T, 1, 1, 64>(plan.per_thread, input, output, rows, cols, stream);
      break;
    case opl::RowPath::kBlock:
      if (vec) launch_block<T, E, kBlockMinV, kBlockMaxV>(plan.per_thread, input, output, rows, cols, stream);
      else if (ragged) launch_block<T, 0, kBlockMinV, kBlockMaxV>(plan.per_thread, input, output, rows, cols, stream);
      else launch_block<T, 1, 16, 64>(plan.per_thread, input, output, rows, cols, stream);
      break;
    case opl::RowPath::kTwoPass:
      softmax_two_pass_kernel<T><<<dim3(rows), dim3(opl::kRowBlockThreads), 0,
                                   stream>>>(input, output, cols, vec ? 1 : 0);
      break;
  }
  return hipGetLastError();
}

}  // namespace

extern "C" int operatorlib_softmax_f32(const float* input, float* output,
                                       int rows, int cols,
                                       void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  return softmax_launch(input, output, rows, cols,
                        static_cast<hipStream_t>(stream_handle));
}

extern "C" int operatorlib_softmax_f16(const operatorlib_half_t* input,
                                       operatorlib_half_t* output, int rows,
                                       int cols, void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  return softmax_launch(reinterpret_cast<const _Float16*>(input),
                        reinterpret_cast<_Float16*>(output), rows, cols,
                        static_cast<hipStream_t>(stream_handle));
}
