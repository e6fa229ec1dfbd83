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

// Ragged rows (hidden % 4 != 0 or unaligned; input and output rows in the
// same 16-byte phase): x and y move as float4 bodies plus scalar head/tail.
// Rows of one launch start at different offsets modulo 16 bytes, so w is
// read per element: from LDS in the wavefront kernel (staged once per
// workgroup of 4 rows), from L2 in the workgroup kernel.
template <int V, int Lanes, typename WeightAt>
__device__ __forceinline__ void ragged_scale_store(
    opl::RaggedRowSlice<V, Lanes>& s, WeightAt w, float* __restrict__ out_row,
    int cols, int t, float inv) {
#pragma unroll
  for (int j = 0; j < V; ++j) {
    if (j * Lanes + t < s.body) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        s.x[4 * j + e] = (s.x[4 * j + e] * inv) * w(s.body_col(t, 4 * j + e));
    }
  }
  const int c = s.extra_col(t, cols);
  if (c >= 0) s.x[4 * V] = (s.x[4 * V] * inv) * w(c);
  s.store(out_row, cols, t);
}

// Copy s (0-3) of the staged weights holds w[c] at float index c + s, so a
// row whose float4 body starts at column `head` reads its weights as
// aligned float4s from copy (4 - head) % 4: conflict-free ds_read_b128
// instead of four 4-byte reads at a 16-byte lane stride.
constexpr int kWeightCopyPitch = opl::kRowWaveMaxCols + 4;

template <int V>
__global__ __launch_bounds__(opl::kRowWaveThreads) void rmsnorm_ragged_wave_kernel(
    const float* __restrict__ input, const float* __restrict__ weight,
    float* __restrict__ output, int rows, int cols, float epsilon) {
  __shared__ __attribute__((aligned(16))) float w_lds[4 * kWeightCopyPitch];
  const int lane = threadIdx.x % opl::kWaveSize;
  const int row = blockIdx.x * opl::kRowWaveRows + threadIdx.x / opl::kWaveSize;
  const bool active = row < rows;  // uniform per wavefront
  const std::size_t offset = static_cast<std::size_t>(active ? row : 0) * cols;
  // Weight loads are issued first and the row's loads right after, so the
  // LDS writes of the weights wait only for the older weight loads and the
  // row's HBM latency overlaps the staging and its barrier.
  constexpr int kWPerThread = opl::kRowWaveMaxCols / opl::kRowWaveThreads;
  float wv[kWPerThread];
#pragma unroll
  for (int i = 0; i < kWPerThread; ++i) {
    const int c = static_cast<int>(threadIdx.x) + opl::kRowWaveThreads * i;
    wv[i] = weight[c < cols ? c : cols - 1];
  }
  opl::RaggedRowSlice<V, opl::kWaveSize> s;
  s.load_raw(input + offset, cols, lane);  // row 0 stands in for inactive waves
  __builtin_amdgcn_sched_barrier(0);       // keep the row's loads in flight
  // Every slot written (those at or past `cols` repeat the last weight and
  // are never read), so the writes need no branches.
#pragma unroll
  for (int copy = 0; copy < 4; ++copy)
#pragma unroll
    for (int i = 0; i < kWPerThread; ++i)
      w_lds[copy * kWeightCopyPitch + copy + static_cast<int>(threadIdx.x) +
            opl::kRowWaveThreads * i] = wv[i];
  __syncthreads();
  if (!active) return;
  s.mask(cols, lane, 0.0f);
  const float ss = opl::wave_reduce<opl::SumOp>(sum_squares(s.x));
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  const int copy = (4 - s.head) & 3;
  const float4* w4 = reinterpret_cast<const float4*>(
      w_lds + copy * kWeightCopyPitch + copy + s.head);  // 16-byte aligned
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int q = j * opl::kWaveSize + lane;
    const float4 wq = w4[q < s.body ? q : 0];
    s.x[4 * j + 0] = (s.x[4 * j + 0] * inv) * wq.x;
    s.x[4 * j + 1] = (s.x[4 * j + 1] * inv) * wq.y;
    s.x[4 * j + 2] = (s.x[4 * j + 2] * inv) * wq.z;
    s.x[4 * j + 3] = (s.x[4 * j + 3] * inv) * wq.w;
  }
  const int c = s.extra_col(lane, cols);
  s.x[4 * V] = (s.x[4 * V] * inv) * w_lds[c >= 0 ? c : 0];
  s.store(output + offset, cols, lane);
}

template <int V>
__global__ __launch_bounds__(opl::kRowBlockThreads) void rmsnorm_ragged_block_kernel(
    const float* __restrict__ input, const float* __restrict__ weight,
    float* __restrict__ output, int cols, float epsilon) {
  __shared__ float slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  opl::RaggedRowSlice<V, opl::kRowBlockThreads> s;
  s.load(input + offset, cols, threadIdx.x, 0.0f);
  const float ss = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(
      sum_squares(s.x), slots);
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  ragged_scale_store(s, [&](int c) { return weight[c]; }, output + offset,
                     cols, threadIdx.x, inv);
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

// W: 4 aligned float4 rows, 1 element-wise, 0 ragged float4 rows.
template <int W, int V, int MaxV>
void launch_wave(int v, const Args& a, hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_wave<W, 2 * V, MaxV>(v, a, stream);
  }
  const int blocks = (a.rows + opl::kRowWaveRows - 1) / opl::kRowWaveRows;
  if constexpr (W == 0)
    rmsnorm_ragged_wave_kernel<V><<<dim3(blocks), dim3(opl::kRowWaveThreads), 0,
                                    stream>>>(a.input, a.weight, a.output,
                                              a.rows, a.cols, a.epsilon);
  else
    rmsnorm_wave_kernel<V, W><<<dim3(blocks), dim3(opl::kRowWaveThreads), 0,
                                stream>>>(a.input, a.weight, a.output, a.rows,
                                          a.cols, a.epsilon);
}

template <int W, int V, int MaxV>
void launch_block(int v, const Args& a, hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_block<W, 2 * V, MaxV>(v, a, stream);
  }
  if constexpr (W == 0)
    rmsnorm_ragged_block_kernel<V><<<dim3(a.rows),
                                     dim3(opl::kRowBlockThreads), 0, stream>>>(
        a.input, a.weight, a.output, a.cols, a.epsilon);
  else
    rmsnorm_block_kernel<V, W><<<dim3(a.rows),
                                 dim3(opl::kRowBlockThreads), 0, stream>>>(
        a.input, a.weight, a.output, a.cols, a.epsilon);
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
  const bool ragged = !vec4 && opl::same_phase16(input, output) &&
                      hidden >= opl::kRaggedMinCols;
  const Args args{input, weight, output, tokens, hidden, epsilon};
  const opl::RowPlan plan = opl::pick_row_plan(hidden, vec4 || ragged);
  switch (plan.path) {
    case opl::RowPath::kWave:
      if (vec4) launch_wave<4, 1, 16>(plan.per_thread, args, stream);
      else if (ragged) launch_wave<0, 1, 16>(plan.per_thread, args, stream);
      else launch_wave<1, 1, 64>(plan.per_thread, args, stream);
      break;
    case opl::RowPath::kBlock:
      if (vec4) launch_block<4, 4, 16>(plan.per_thread, args, stream);
      else if (ragged) launch_block<0, 4, 16>(plan.per_thread, args, stream);
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
