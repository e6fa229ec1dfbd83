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
