// softmax_f32: numerically stable softmax over the last dimension of a
// row-major [rows, cols] fp32 matrix.
//
// Reference: operatorlib::softmax_f32 (src/softmax.cu:182-202) with three
// CUDA kernels (:52-176); its general path reads the input twice and the
// output twice. Same maths here:
//   m = max_c x[c];  p[c] = exp(x[c] - m);  out[c] = p[c] * (1 / sum_c p[c])
// with exp evaluated as exp2((x - m) * log2 e) on v_exp_f32.
//
// MI355X design: the row stays in VGPRs between the max, exp/sum and scale
// steps, so every path up to 32768 columns reads x once and writes once
// (the HBM minimum, 8 bytes per element). Reductions are wave64 DPP
// butterflies (plus an 8-slot LDS combine for workgroup rows). Rows longer
// than 32768 columns use an online (max, sum) first pass and re-read x once.
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

template <int V, int W>
__global__ __launch_bounds__(opl::kRowWaveThreads) void softmax_wave_kernel(
    const float* __restrict__ input, float* __restrict__ output, int rows,
    int cols) {
  const int lane = threadIdx.x % opl::kWaveSize;
  const int row = blockIdx.x * opl::kRowWaveRows + threadIdx.x / opl::kWaveSize;
  if (row >= rows) return;  // uniform per wavefront
  const std::size_t offset = static_cast<std::size_t>(row) * cols;
  typename opl::SliceFor<V, opl::kWaveSize, W>::type s;
  s.load(input + offset, cols, lane, -INFINITY);
  const float m = opl::wave_reduce<opl::MaxOp>(local_max(s.x));
  const float sum = opl::wave_reduce<opl::SumOp>(exp_shift_sum(s.x, m));
  scale(s.x, 1.0f / sum);
  s.store(output + offset, cols, lane);
}

template <int V, int W>
__global__ __launch_bounds__(opl::kRowBlockThreads) void softmax_block_kernel(
    const float* __restrict__ input, float* __restrict__ output, int cols) {
  __shared__ float max_slots[opl::kRowBlockWaves];
  __shared__ float sum_slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  typename opl::SliceFor<V, opl::kRowBlockThreads, W>::type s;
  s.load(input + offset, cols, threadIdx.x, -INFINITY);
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

__global__ __launch_bounds__(opl::kRowBlockThreads) void softmax_two_pass_kernel(
    const float* __restrict__ input, float* __restrict__ output, int cols,
    int vec4) {
  __shared__ float max_slots[opl::kRowBlockWaves];
  __shared__ float sum_slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  const float* row = input + offset;
  float* out = output + offset;
  const int t = threadIdx.x;
  constexpr int kT = opl::kRowBlockThreads;
  float m = -FLT_MAX;
  float s = 0.0f;
  if (vec4) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    for (int i = t; i < cols / 4; i += kT) {
      const float4 q = r4[i];
      online_update(q.x, m, s);
      online_update(q.y, m, s);
      online_update(q.z, m, s);
      online_update(q.w, m, s);
    }
  } else {
    for (int c = t; c < cols; c += kT) online_update(row[c], m, s);
  }
  const float row_max =
      opl::block_reduce<opl::MaxOp, opl::kRowBlockWaves>(m, max_slots);
  const float row_sum = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(
      s * opl::fast_exp2((m - row_max) * kLog2e), sum_slots);
  const float inv = 1.0f / row_sum;
  if (vec4) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    float4* o4 = reinterpret_cast<float4*>(out);
    for (int i = t; i < cols / 4; i += kT) {
      const float4 q = r4[i];
      o4[i] = make_float4(
          opl::fast_exp2((q.x - row_max) * kLog2e) * inv,
          opl::fast_exp2((q.y - row_max) * kLog2e) * inv,
          opl::fast_exp2((q.z - row_max) * kLog2e) * inv,
          opl::fast_exp2((q.w - row_max) * kLog2e) * inv);
    }
  } else {
    for (int c = t; c < cols; c += kT)
      out[c] = opl::fast_exp2((row[c] - row_max) * kLog2e) * inv;
  }
}

// Launches the kernel instance whose per-thread count V is the smallest power
// of two >= v (v comes from pick_row_plan, so it never exceeds MaxV).
template <int W, int V, int MaxV>
void launch_wave(int v, const float* in, float* out, int rows, int cols,
                 hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_wave<W, 2 * V, MaxV>(v, in, out, rows, cols, stream);
  }
  const int blocks = (rows + opl::kRowWaveRows - 1) / opl::kRowWaveRows;
  softmax_wave_kernel<V, W><<<dim3(blocks), dim3(opl::kRowWaveThreads), 0,
                              stream>>>(in, out, rows, cols);
}

template <int W, int V, int MaxV>
void launch_block(int v, const float* in, float* out, int rows, int cols,
                  hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_block<W, 2 * V, MaxV>(v, in, out, rows, cols, stream);
  }
  softmax_block_kernel<V, W><<<dim3(rows), dim3(opl::kRowBlockThreads),
                               0, stream>>>(in, out, cols);
}

}  // namespace

extern "C" int operatorlib_softmax_f32(const float* input, float* output,
                                       int rows, int cols,
                                       void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  hipStream_t stream = static_cast<hipStream_t>(stream_handle);
  const bool vec4 =
      cols % 4 == 0 && opl::aligned16(input) && opl::aligned16(output);
  // Ragged rows (cols % 4 != 0 or unaligned) keep 16-byte accesses when
  // input and output rows share their 16-byte phase.
  const bool ragged = !vec4 && opl::same_phase16(input, output) &&
                      cols >= opl::kRaggedMinCols;
  const opl::RowPlan plan = opl::pick_row_plan(cols, vec4 || ragged);
  switch (plan.path) {
    case opl::RowPath::kWave:
      if (vec4) launch_wave<4, 1, 16>(plan.per_thread, input, output, rows, cols, stream);
      else if (ragged) launch_wave<0, 1, 16>(plan.per_thread, input, output, rows, cols, stream);
      else launch_wave<1, 1, 64>(plan.per_thread, input, output, rows, cols, stream);
      break;
    case opl::RowPath::kBlock:
      if (vec4) launch_block<4, 4, 16>(plan.per_thread, input, output, rows, cols, stream);
      else if (ragged) launch_block<0, 4, 16>(plan.per_thread, input, output, rows, cols, stream);
      else launch_block<1, 16, 64>(plan.per_thread, input, output, rows, cols, stream);
      break;
    case opl::RowPath::kTwoPass:
      softmax_two_pass_kernel<<<dim3(rows), dim3(opl::kRowBlockThreads), 0,
                                stream>>>(input, output, cols, vec4 ? 1 : 0);
      break;
  }
  return hipGetLastError();
}
