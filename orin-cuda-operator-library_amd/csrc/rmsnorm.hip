// rmsnorm_f32 / rmsnorm_f16: y[t, h] = x[t, h] * rsqrt(mean_h(x[t, :]^2) +
// eps) * w[h]. The fp16 variant (fp16 x, w and y) computes in fp32 and
// rounds y to fp16 once, on store: the "FP16 input, FP32 accumulation"
// extension the reference defers (docs/pytorch_extension.md:143-146).
//
// Reference: operatorlib::rmsnorm_f32 (src/rmsnorm.cu:77-95, kernels :27-71).
// Its kernels read x twice (once for the sum of squares, once to scale).
// Same maths and rounding order here: inv = rsqrt(ss / hidden + eps) in fp32,
// y = (x * inv) * w.
//
// MI355X design: a single fused pass. The row is held in VGPRs (one
// wavefront per row up to 4096 columns, one 512-thread workgroup per row up
// to 32768), so x is read from HBM once and y written once; w (one row of
// bytes) is shared by all rows and served from L2/MALL after first touch.
// Algorithmic traffic: (2 * tokens * hidden + hidden) * sizeof(element).
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

template <int V, int Lanes, int W, typename T>
__device__ __forceinline__ void scale_store(
    opl::RowSlice<V, Lanes, W, T>& s, const T* __restrict__ weight,
    T* __restrict__ out_row, int cols, int t, float inv) {
  opl::RowSlice<V, Lanes, W, T> w;
  w.load(weight, cols, t, 0.0f);
#pragma unroll
  for (int i = 0; i < opl::RowSlice<V, Lanes, W, T>::kCount; ++i)
    s.x[i] = (s.x[i] * inv) * w.x[i];
  s.store(out_row, cols, t);
}

template <typename T, int V, int W>
__global__ __launch_bounds__(opl::kRowWaveThreads) void rmsnorm_wave_kernel(
    const T* __restrict__ input, const T* __restrict__ weight,
    T* __restrict__ output, int rows, int cols, float epsilon) {
  const int lane = threadIdx.x % opl::kWaveSize;
  const int row = blockIdx.x * opl::kRowWaveRows + threadIdx.x / opl::kWaveSize;
  if (row >= rows) return;  // uniform per wavefront
  const std::size_t offset = static_cast<std::size_t>(row) * cols;
  opl::RowSlice<V, opl::kWaveSize, W, T> s;
  s.template load<true>(input + offset, cols, lane, 0.0f);
  const float ss = opl::wave_reduce<opl::SumOp>(sum_squares(s.x));
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  scale_store(s, weight, output + offset, cols, lane, inv);
}

template <typename T, int V, int W>
__global__ __launch_bounds__(opl::kRowBlockThreads) void rmsnorm_block_kernel(
    const T* __restrict__ input, const T* __restrict__ weight,
    T* __restrict__ output, int cols, float epsilon) {
  __shared__ float slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  opl::RowSlice<V, opl::kRowBlockThreads, W, T> s;
  s.template load<true>(input + offset, cols, threadIdx.x, 0.0f);
  const float ss = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(
      sum_squares(s.x), slots);
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  scale_store(s, weight, output + offset, cols, threadIdx.x, inv);
}

// Ragged rows (hidden % E != 0 or unaligned; input and output rows in the
// same 16-byte phase): x and y move as 16-byte chunk bodies plus scalar
// head/tail. Rows of one launch start at different offsets modulo 16 bytes,
// so w is read per element: from LDS in the wavefront kernel (staged once
// per workgroup of 4 rows), from L2 in the workgroup kernel.
template <int V, int Lanes, typename T, typename WeightAt>
__device__ __forceinline__ void ragged_scale_store(
    opl::RaggedRowSlice<V, Lanes, T>& s, WeightAt w, T* __restrict__ out_row,
    int cols, int t, float inv) {
  constexpr int E = opl::RaggedRowSlice<V, Lanes, T>::kE;
  // All weight reads issue before the first use (clamped to column 0 for
  // slots outside the row, whose results store() never writes).
  float wv[E * V + 1];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const bool in = j * Lanes + t < s.body;
#pragma unroll
    for (int e = 0; e < E; ++e) wv[E * j + e] = w(in ? s.body_col(t, E * j + e) : 0);
  }
  const int c = s.extra_col(t, cols);
  wv[E * V] = w(c >= 0 ? c : 0);
#pragma unroll
  for (int i = 0; i < E * V + 1; ++i) s.x[i] = (s.x[i] * inv) * wv[i];
  s.store(out_row, cols, t);
}

// The wavefront kernel stages E shifted copies of the weights (E elements
// per 16-byte chunk): copy s holds w[c] at element index c + s, so a row
// whose chunk body starts at column `head` reads its weights as aligned
// 16-byte chunks from copy (E - head) % E: conflict-free ds_read_b128
// instead of E narrow reads at a 16-byte lane stride.
template <typename T>
constexpr int weight_copy_pitch() {
  return opl::kRowWaveMaxCols + opl::RowElem<T>::kPerChunk;
}

template <typename T, int V>
__global__ __launch_bounds__(opl::kRowWaveThreads) void rmsnorm_ragged_wave_kernel(
    const T* __restrict__ input, const T* __restrict__ weight,
    T* __restrict__ output, int rows, int cols, float epsilon) {
  using Chunk = typename opl::RowElem<T>::Chunk;
  constexpr int E = opl::RowElem<T>::kPerChunk;
  constexpr int kPitch = weight_copy_pitch<T>();
  __shared__ __attribute__((aligned(16))) T w_lds[E * kPitch];
  const int lane = threadIdx.x % opl::kWaveSize;
  const int row = blockIdx.x * opl::kRowWaveRows + threadIdx.x / opl::kWaveSize;
  const bool active = row < rows;  // uniform per wavefront
  const std::size_t offset = static_cast<std::size_t>(active ? row : 0) * cols;
  // Weight loads are issued first and the row's loads right after, so the
  // LDS writes of the weights wait only for the older weight loads and the
  // row's HBM latency overlaps the staging and its barrier.
  constexpr int kWPerThread = opl::kRowWaveMaxCols / opl::kRowWaveThreads;
  T wv[kWPerThread];
#pragma unroll
  for (int i = 0; i < kWPerThread; ++i) {
    const int c = static_cast<int>(threadIdx.x) + opl::kRowWaveThreads * i;
    wv[i] = weight[c < cols ? c : cols - 1];
  }
  opl::RaggedRowSlice<V, opl::kWaveSize, T> s;
  s.template load_raw<true>(input + offset, cols, lane);  // row 0 stands in for inactive waves
  __builtin_amdgcn_sched_barrier(0);       // keep the row's loads in flight
  // Every slot written (those at or past `cols` repeat the last weight and
  // are never read), so the writes need no branches.
#pragma unroll
  for (int copy = 0; copy < E; ++copy)
#pragma unroll
    for (int i = 0; i < kWPerThread; ++i)
      w_lds[copy * kPitch + copy + static_cast<int>(threadIdx.x) +
            opl::kRowWaveThreads * i] = wv[i];
  __syncthreads();
  if (!active) return;
  s.mask(cols, lane, 0.0f);
  const float ss = opl::wave_reduce<opl::SumOp>(sum_squares(s.x));
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  const int copy = (E - s.head) & (E - 1);
  const Chunk* wc = reinterpret_cast<const Chunk*>(
      w_lds + copy * kPitch + copy + s.head);  // 16-byte aligned
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int q = j * opl::kWaveSize + lane;
    const Chunk wq = wc[q < s.body ? q : 0];
#pragma unroll
    for (int e = 0; e < E; ++e)
      s.x[E * j + e] = (s.x[E * j + e] * inv) * static_cast<float>(wq[e]);
  }
  const int c = s.extra_col(lane, cols);
  s.x[E * V] = (s.x[E * V] * inv) * static_cast<float>(w_lds[c >= 0 ? c : 0]);
  s.store(output + offset, cols, lane);
}

template <typename T, int V>
__global__ __launch_bounds__(opl::kRowBlockThreads) void rmsnorm_ragged_block_kernel(
    const T* __restrict__ input, const T* __restrict__ weight,
    T* __restrict__ output, int cols, float epsilon) {
  __shared__ float slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  opl::RaggedRowSlice<V, opl::kRowBlockThreads, T> s;
  s.template load<true>(input + offset, cols, threadIdx.x, 0.0f);
  const float ss = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(
      sum_squares(s.x), slots);
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  ragged_scale_store(
      s, [&](int c) { return static_cast<float>(weight[c]); },
      output + offset, cols, threadIdx.x, inv);
}

template <typename T>
__global__ __launch_bounds__(opl::kRowBlockThreads) void rmsnorm_two_pass_kernel(
    const T* __restrict__ input, const T* __restrict__ weight,
    T* __restrict__ output, int cols, float epsilon) {
  __shared__ float slots[opl::kRowBlockWaves];
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols;
  const T* row = input + offset;
  T* out = output + offset;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < cols; c += opl::kRowBlockThreads) {
    const float x = static_cast<float>(row[c]);
    ss += x * x;
  }
  ss = opl::block_reduce<opl::SumOp, opl::kRowBlockWaves>(ss, slots);
  const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
  for (int c = threadIdx.x; c < cols; c += opl::kRowBlockThreads)
    out[c] = static_cast<T>((static_cast<float>(row[c]) * inv) *
                            static_cast<float>(weight[c]));
}

template <typename T>
struct Args {
  const T* input;
  const T* weight;
  T* output;
  int rows;
  int cols;
  float epsilon;
};

// W: E aligned 16-byte chunks, 1 element-wise, 0 ragged chunk rows.
template <typename T, int W, int V, int MaxV>
void launch_wave(int v, const Args<T>& a, hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_wave<T, W, 2 * V, MaxV>(v, a, stream);
  }
  const int blocks = (a.rows + opl::kRowWaveRows - 1) / opl::kRowWaveRows;
  if constexpr (W == 0)
    rmsnorm_ragged_wave_kernel<T, V><<<dim3(blocks), dim3(opl::kRowWaveThreads),
                                       0, stream>>>(a.input, a.weight, a.output,
                                                    a.rows, a.cols, a.epsilon);
  else
    rmsnorm_wave_kernel<T, V, W><<<dim3(blocks), dim3(opl::kRowWaveThreads), 0,
                                   stream>>>(a.input, a.weight, a.output, a.rows,
                                             a.cols, a.epsilon);
}

template <typename T, int W, int V, int MaxV>
void launch_block(int v, const Args<T>& a, hipStream_t stream) {
  if constexpr (V < MaxV) {
    if (v > V) return launch_block<T, W, 2 * V, MaxV>(v, a, stream);
  }
  if constexpr (W == 0)
    rmsnorm_ragged_block_kernel<T, V><<<dim3(a.rows),
                                        dim3(opl::kRowBlockThreads), 0, stream>>>(
        a.input, a.weight, a.output, a.cols, a.epsilon);
  else
    rmsnorm_block_kernel<T, V, W><<<dim3(a.rows),
                                    dim3(opl::kRowBlockThreads), 0, stream>>>(
        a.input, a.weight, a.output, a.cols, a.epsilon);
}

// Shared dispatch of the fp32 and fp16 entry points (E elements per 16-byte
// chunk; per-thread counts as in softmax).
template <typename T>
int rmsnorm_launch(const Args<T>& args, hipStream_t stream) {
  constexpr int E = opl::RowElem<T>::kPerChunk;
  constexpr int kWaveMaxV = opl::kRowWaveMaxCols / (opl::kWaveSize * E);
  constexpr int kBlockMinV =
      2 * opl::kRowWaveMaxCols / (opl::kRowBlockThreads * E);
  constexpr int kBlockMaxV =
      opl::kRowBlockMaxCols / (opl::kRowBlockThreads * E);
  const int hidden = args.cols;
  const bool vec = hidden % E == 0 && opl::aligned16(args.input) &&
                   opl::aligned16(args.weight) && opl::aligned16(args.output);
  const bool ragged =
      !vec && opl::same_phase16(args.input, args.output) &&
      hidden >= opl::RaggedRowSlice<1, opl::kWaveSize, T>::kMinCols;
  const opl::RowPlan plan = opl::pick_row_plan(hidden, vec || ragged ? E : 1);
  switch (plan.path) {
    case opl::RowPath::kWave:
      if (vec) launch_wave<T, E, 1, kWaveMaxV>(plan.per_thread, args, stream);
      else if (ragged) launch_wave<T, 0, 1, kWaveMaxV>(plan.per_thread, args, stream);
      else launch_wave<T, 1, 1, 64>(plan.per_thread, args, stream);
      break;
    case opl::RowPath::kBlock:
      if (vec) launch_block<T, E, kBlockMinV, kBlockMaxV>(plan.per_thread, args, stream);
      else if (ragged) launch_block<T, 0, kBlockMinV, kBlockMaxV>(plan.per_thread, args, stream);
      else launch_block<T, 1, 16, 64>(plan.per_thread, args, stream);
      break;
    case opl::RowPath::kTwoPass:
      rmsnorm_two_pass_kernel<T><<<dim3(args.rows), dim3(opl::kRowBlockThreads),
                                   0, stream>>>(args.input, args.weight,
                                                args.output, hidden,
                                                args.epsilon);
      break;
  }
  return hipGetLastError();
}

}  // namespace

extern "C" int operatorlib_rmsnorm_f32(const float* input, const float* weight,
                                       float* output, int tokens, int hidden,
                                       float epsilon, void* stream_handle) {
  if (!opl::rmsnorm_args_ok(input, weight, output, tokens, hidden, epsilon))
    return hipErrorInvalidValue;
  return rmsnorm_launch(
      Args<float>{input, weight, output, tokens, hidden, epsilon},
      static_cast<hipStream_t>(stream_handle));
}

extern "C" int operatorlib_rmsnorm_f16(const operatorlib_half_t* input,
                                       const operatorlib_half_t* weight,
                                       operatorlib_half_t* output, int tokens,
                                       int hidden, float epsilon,
                                       void* stream_handle) {
  if (!opl::rmsnorm_args_ok(input, weight, output, tokens, hidden, epsilon))
    return hipErrorInvalidValue;
  return rmsnorm_launch(
      Args<_Float16>{reinterpret_cast<const _Float16*>(input),
                     reinterpret_cast<const _Float16*>(weight),
                     reinterpret_cast<_Float16*>(output), tokens, hidden,
                     epsilon},
      static_cast<hipStream_t>(stream_handle));
}
