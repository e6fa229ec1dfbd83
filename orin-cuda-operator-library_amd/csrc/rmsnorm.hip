// rmsnorm_f32: y[t, h] = x[t, h] * rsqrt(mean_h(x[t, :]^2) + eps) * w[h].
//
// Reference: operatorlib::rmsnorm_f32 (src/rmsnorm.cu:77-95, kernels :27-71).
// Its kernels read x twice (once for the sum of squares, once to scale).
// Same maths and rounding order here: inv = rsqrt(ss / hidden + eps) in fp32,
// y = (x * inv) * w.
//
// MI355X design: a single fused pass. The row is held in VGPRs (one
// wavefront per row up to 4096 columns, one 512-thread workgroup per row up
// to 32768), so x is read from HBM once and y written once; w (hidden * 4
// bytes) is shared by all rows and served from L2/MALL after first touch.
// Algorithmic traffic: (2 * tokens * hidden + hidden) * 4 bytes.
// Only rows longer than 32768 columns re-read x (two passes).

#include <hip/hip_runtime.h>

#include <cstddef>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "rowwise.hpp"
#include "validate.hpp"

namespace {

template <int N>
__device__ __forceinline__ float sum_squares(const float (&x)[N]) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) s += x[i] * x[i];
  return s;
}

template <int V, int Lanes, int W>
__device__ __forceinline__ void scale_store(
    opl::RowSlice<V, Lanes, W>& s, const float* __restrict__ weight,
    float* __restrict__ out_row, int cols, int t, float inv) {
  opl::RowSlice<V, Lanes, W> w;
  w.load(weight, cols, t, 0.0f);
#pragma unroll
  for (int i = 0; i < opl::RowSlice<V, Lanes, W>::kCount; ++i)
    s.x[i] = (s.x[i] * inv) * w.x[i];
  s.store(out_row, cols, t);
}

template <int V, int W>
__global__ __launch_bounds__(opl::kRowWaveThreads) void rmsnorm_wave_kernel(
    const float* __restrict__ input, const float* __restrict__ weight,
    float* __restrict__ output, int rows, int cols, float epsilon) {
  const int lane = threadIdx.x % opl::kWaveSize;
  const int row = blockIdx.x * opl::kRowWaveRows + threadIdx.x / opl::kWaveSize;
  if (row >= rows) return;  // uniform per wavefront
  const std::size_t offset = static_cast<std::size_t>(row) * cols;
  opl::RowSlice<V, opl::kWaveSize, W> s;
  s.load(input + offset, cols, lane, 0.0f);
  const float ss = opl::wave_reduce<opl::SumOp>(sum_squares(s.x));
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  scale_store(s, weight, output + offset, cols, lane, inv);
}

template <int V, int W>
__global__ __launch_bounds__(opl::kRowBlockThreads) void rmsnorm_block_kernel(
    const float* __restrict__ input, const float* __restrict__ weight,
    float* __restrict__ output, int cols, float epsilon) {
  __shared__ float slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  opl::RowSlice<V, opl::kRowBlockThreads, W> s;
  s.load(input + offset, cols, threadIdx.x, 0.0f);
  const float ss = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(
      sum_squares(s.x), slots);
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  scale_store(s, weight, output + offset, cols, threadIdx.x, inv);
}

__global__ __launch_bounds__(opl::kRowBlockThreads) void rmsnorm_two_pass_kernel(
    const float* __restrict__ input, const float* __restrict__ weight,
    float* __restrict__ output, int cols, float epsilon) {
  __shared__ float slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  const float* row = input + offset;
  float* out = output + offset;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < cols; c += opl::kRowBlockThreads)
    ss += row[c] * row[c];
  ss = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(ss, slots);
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  for (int c = threadIdx.x; c < cols; c += opl::kRowBlockThreads)
    out[c] = (row[c] * inv) * weight[c];
}

struct Args {
  const float* input;
  const float* weight;
  float* output;
  int rows;
  int cols;
  float epsilon;
};

template <int W, int V, int MaxV>
void launch_wave(int v, const Args& a, hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_wave<W, 2 * V, MaxV>(v, a, stream);
  }
  const int blocks = (a.rows + opl::kRowWaveRows - 1) / opl::kRowWaveRows;
  rmsnorm_wave_kernel<V, W><<<dim3(blocks), dim3(opl::kRowWaveThreads), 0,
                              stream>>>(a.input, a.weight, a.output, a.rows,
                                        a.cols, a.epsilon);
}

template <int W, int V, int MaxV>
void launch_block(int v, const Args& a, hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_block<W, 2 * V, MaxV>(v, a, stream);
  }
  rmsnorm_block_kernel<V, W><<<dim3(a.rows), dim3(opl::kRowBlockThreads), 0,
                               stream>>>(a.input, a.weight, a.output, a.cols,
                                         a.epsilon);
}

}  // namespace

extern "C" int operatorlib_rmsnorm_f32(const float* input, const float* weight,
                                       float* output, int tokens, int hidden,
                                       float epsilon, void* stream_handle) {
  if (!opl::rmsnorm_args_ok(input, weight, output, tokens, hidden, epsilon))
    return hipErrorInvalidValue;
  hipStream_t stream = static_cast<hipStream_t>(stream_handle);
  const bool vec4 = hidden % 4 == 0 && opl::aligned16(input) &&
                    opl::aligned16(weight) && opl::aligned16(output);
  const Args args{input, weight, output, tokens, hidden, epsilon};
  const opl::RowPlan plan = opl::pick_row_plan(hidden, vec4);
  switch (plan.path) {
    case opl::RowPath::kWave:
      if (vec4) launch_wave<4, 1, 16>(plan.per_thread, args, stream);
      else launch_wave<1, 1, 64>(plan.per_thread, args, stream);
      break;
    case opl::RowPath::kBlock:
      if (vec4) launch_block<4, 4, 16>(plan.per_thread, args, stream);
      else launch_block<1, 16, 64>(plan.per_thread, args, stream);
      break;
    case opl::RowPath::kTwoPass:
      rmsnorm_two_pass_kernel<<<dim3(tokens), dim3(opl::kRowBlockThreads), 0,
                                stream>>>(input, weight, output, hidden,
                                          epsilon);
      break;
  }
  return hipGetLastError();
}
