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
// Rows longer than 32768 columns, and a few long rows that would leave CUs
// idle, are cut into segments over workgroups: an online (max, sum) pass
// per segment, then a pass that combines the row's pairs, re-reads x once
// and writes.
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
#include "scratch.hpp"
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

// Short rows: a group of G lanes per row, 64 / G rows per wavefront, one
// access per lane: W = E (16-byte chunk t of the row; cols % E == 0 and
// aligned rows) or W = 1 (element t, any shape). A wavefront per row left
// most lanes idle here (1048576 x 8: 135 us against a 10 us copy of the
// same bytes). Wavefronts stride over blocks of rows, U blocks in flight.
using opl::kGroupMaxBlocks;
using opl::kGroupThreads;

template <typename T, int G, int W, int U>
__global__ __launch_bounds__(kGroupThreads) void softmax_group_kernel(
    const T* __restrict__ input, T* __restrict__ output, int rows, int cols) {
  using A = typename opl::Access<T, W>::type;
  constexpr int kRowsPerWave = opl::kWaveSize / G;
  constexpr int kWaves = kGroupThreads / opl::kWaveSize;
  const int lane = threadIdx.x % opl::kWaveSize;
  const int t = lane % G;
  const int r_lane = lane / G;
  const bool lane_in = t * W < cols;
  const long long stride = static_cast<long long>(gridDim.x) * kWaves * kRowsPerWave * U;
  for (long long r0 = (static_cast<long long>(blockIdx.x) * kWaves + threadIdx.x / opl::kWaveSize) *
                      kRowsPerWave * U;
       r0 < rows; r0 += stride) {
    A q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long row = r0 + u * kRowsPerWave + r_lane;
      const bool in = lane_in && row < rows;
      q[u] = __builtin_nontemporal_load(
          reinterpret_cast<const A*>(input + (in ? row * cols + t * W : 0)));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long row = r0 + u * kRowsPerWave + r_lane;
      const bool in = lane_in && row < rows;
      float x[W];
#pragma unroll
      for (int e = 0; e < W; ++e) x[e] = in ? static_cast<float>(q[u][e]) : -INFINITY;
      const float m = opl::group_reduce<opl::MaxOp, G>(local_max(x));
      const float inv = 1.0f / opl::group_reduce<opl::SumOp, G>(exp_shift_sum(x, m));
      if (in) {
        A y;
#pragma unroll
        for (int e = 0; e < W; ++e) y[e] = static_cast<T>(x[e] * inv);
        __builtin_nontemporal_store(y, reinterpret_cast<A*>(output + row * cols + t * W));
      }
    }
  }
}

template <typename T, int W, int U, int G = 1>
void launch_group(int g, const T* in, T* out, int rows, int cols, hipStream_t stream) {
  if constexpr (G < 32) {
    if (g > G) return launch_group<T, W, U, 2 * G>(g, in, out, rows, cols, stream);
  }
  constexpr int kRowsPerBlock = kGroupThreads / G * U;
  const long long blocks = (static_cast<long long>(rows) + kRowsPerBlock - 1) / kRowsPerBlock;
  softmax_group_kernel<T, G, W, U>
      <<<dim3(static_cast<unsigned>(blocks < kGroupMaxBlocks ? blocks : kGroupMaxBlocks)),
         dim3(kGroupThreads), 0, stream>>>(in, out, rows, cols);
}

// Rows over several workgroups (opl::split_plan picks them: rows too long
// for registers, and few long rows, where one workgroup per row left most
// CUs idle: 32 x 50257 took 34.5 us, 1 x 2^20 357 us). Pass 1 writes every
// segment's (max, sum of exp(x - max)) to scratch; pass 2 combines the
// row's pairs in segment order (every wavefront of the row computes the
// same bits), re-reads its segment (from the caches at these sizes) and
// writes exp(x - max) / sum. Segments walk their elements with 16-byte
// accesses at any alignment (opl::Segment).
using opl::kSplitThreads;
using opl::kSplitUnroll;
using opl::kSplitWaves;
using opl::SplitPlan;

inline std::size_t split_bytes(int rows, const SplitPlan& p) {
  return p.segments > 0 ? sizeof(float2) * static_cast<std::size_t>(rows) * p.segments : 0;
}

// (m, s) <- running max and sum of exp(x - m) after the values x[0..N).
template <int N>
__device__ __forceinline__ void online_block(const float (&x)[N], float& m, float& s) {
  const float nm = fmaxf(m, local_max(x));
  s *= opl::fast_exp2((m - nm) * kLog2e);
#pragma unroll
  for (int e = 0; e < N; ++e) s += opl::fast_exp2((x[e] - nm) * kLog2e);
  m = nm;
}

template <typename T>
__global__ __launch_bounds__(kSplitThreads) void softmax_split_stats_kernel(
    const T* __restrict__ input, float2* __restrict__ partials, int cols, int seg_len) {
  using Chunk = typename opl::RowElem<T>::Chunk;
  constexpr int E = opl::RowElem<T>::kPerChunk;
  __shared__ float max_slots[kSplitWaves];
  __shared__ float sum_slots[kSplitWaves];
  const int c0 = blockIdx.y * seg_len;
  const int n = min(cols - c0, seg_len);
  const T* p = input + static_cast<std::size_t>(blockIdx.x) * cols + c0;
  const opl::Segment<T> sg(p, n);
  const Chunk* body = reinterpret_cast<const Chunk*>(p + sg.head);
  const int t = threadIdx.x;
  // -FLT_MAX, not -inf: a thread with no elements, or only -inf ones,
  // keeps s = 0 through every rescale.
  float m = -FLT_MAX, s = 0.0f;
  for (int i0 = t; i0 < sg.body; i0 += kSplitThreads * kSplitUnroll) {
    Chunk q[kSplitUnroll];
#pragma unroll
    for (int u = 0; u < kSplitUnroll; ++u) {
      const int i = i0 + u * kSplitThreads;
      q[u] = body[i < sg.body ? i : i0];  // cached: pass 2 reads it again
    }
#pragma unroll
    for (int u = 0; u < kSplitUnroll; ++u) {
      if (i0 + u * kSplitThreads < sg.body) {
        float x[E];
#pragma unroll
        for (int e = 0; e < E; ++e) x[e] = static_cast<float>(q[u][e]);
        online_block(x, m, s);
      }
    }
  }
  const int xc = sg.extra(t);
  if (xc >= 0) {
    const float x[1] = {static_cast<float>(p[xc])};
    online_block(x, m, s);
  }
  const float seg_max = opl::block_reduce<opl::MaxOp, kSplitWaves>(m, max_slots);
  const float seg_sum = opl::block_reduce<opl::SumOp, kSplitWaves>(
      s * opl::fast_exp2((m - seg_max) * kLog2e), sum_slots);
  if (t == 0)
    partials[static_cast<std::size_t>(blockIdx.x) * gridDim.y + blockIdx.y] =
        make_float2(seg_max, seg_sum);
}

// kChunks: input and output rows share their 16-byte phase (16-byte
// accesses on both sides); otherwise element accesses.
template <typename T, bool kChunks>
__global__ __launch_bounds__(kSplitThreads) void softmax_split_apply_kernel(
    const T* __restrict__ input, T* __restrict__ output,
    const float2* __restrict__ partials, int cols, int seg_len) {
  using Chunk = typename opl::RowElem<T>::Chunk;
  constexpr int E = opl::RowElem<T>::kPerChunk;
  const int segments = gridDim.y;
  const float2* pr = partials + static_cast<std::size_t>(blockIdx.x) * segments;
  const int lane = threadIdx.x % opl::kWaveSize;
  float pm = -FLT_MAX;
  for (int i = lane; i < segments; i += opl::kWaveSize) pm = fmaxf(pm, pr[i].x);
  const float row_max = opl::wave_reduce<opl::MaxOp>(pm);
  float ps = 0.0f;
  for (int i = lane; i < segments; i += opl::kWaveSize)
    ps += pr[i].y * opl::fast_exp2((pr[i].x - row_max) * kLog2e);
  const float inv = 1.0f / opl::wave_reduce<opl::SumOp>(ps);
  auto f = [&](float x) { return opl::fast_exp2((x - row_max) * kLog2e) * inv; };

  const int c0 = blockIdx.y * seg_len;
  const int n = min(cols - c0, seg_len);
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols + c0;
  const T* p = input + offset;
  T* o = output + offset;
  const int t = threadIdx.x;
  if constexpr (kChunks) {
    const opl::Segment<T> sg(p, n);
    const Chunk* body = reinterpret_cast<const Chunk*>(p + sg.head);
    Chunk* obody = reinterpret_cast<Chunk*>(o + sg.head);
    for (int i0 = t; i0 < sg.body; i0 += kSplitThreads * kSplitUnroll) {
      Chunk q[kSplitUnroll];
#pragma unroll
      for (int u = 0; u < kSplitUnroll; ++u) {
        const int i = i0 + u * kSplitThreads;
        q[u] = __builtin_nontemporal_load(body + (i < sg.body ? i : i0));
      }
#pragma unroll
      for (int u = 0; u < kSplitUnroll; ++u) {
        const int i = i0 + u * kSplitThreads;
        if (i < sg.body) {
          Chunk y;
#pragma unroll
          for (int e = 0; e < E; ++e) y[e] = static_cast<T>(f(static_cast<float>(q[u][e])));
          __builtin_nontemporal_store(y, obody + i);
        }
      }
    }
    const int xc = sg.extra(t);
    if (xc >= 0) o[xc] = static_cast<T>(f(static_cast<float>(p[xc])));
  } else {
    constexpr int U = 2 * kSplitUnroll;
    for (int i0 = t; i0 < n; i0 += kSplitThreads * U) {
      T q[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kSplitThreads;
        q[u] = __builtin_nontemporal_load(p + (i < n ? i : i0));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kSplitThreads;
        if (i < n) __builtin_nontemporal_store(static_cast<T>(f(static_cast<float>(q[u]))), o + i);
      }
    }
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
                   const opl::ScratchSource& src, hipStream_t stream) {
  constexpr int E = opl::RowElem<T>::kPerChunk;
  constexpr int kWaveMaxV = opl::kRowWaveMaxCols / (opl::kWaveSize * E);
  constexpr int kBlockMinV =
      2 * opl::kRowWaveMaxCols / (opl::kRowBlockThreads * E);
  constexpr int kBlockMaxV =
      opl::kRowBlockMaxCols / (opl::kRowBlockThreads * E);
  const SplitPlan split = opl::split_plan(rows, cols);
  const std::size_t bytes = split_bytes(rows, split);
  if (src.workspace_mode && !opl::workspace_ok(src.data, src.bytes, bytes))
    return hipErrorInvalidValue;
  if (split.segments > 0) {
    // 8 bytes per (row, segment): fewer than 2 * kSplitTargetBlocks pairs
    // for split rows, one per row otherwise (a matrix that fits in HBM has
    // far fewer rows than the arena holds pairs).
    opl::ScratchLease lease(stream, src.workspace_mode ? src.data : nullptr, src.bytes);
    if (lease.status() != hipSuccess) return lease.status();
    float2* partials = static_cast<float2*>(lease.data());
    // rows on x (up to 2^31 - 1), segments (at most 512) on y
    const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(split.segments));
    softmax_split_stats_kernel<T><<<grid, dim3(kSplitThreads), 0, stream>>>(
        input, partials, cols, split.seg_len);
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) return status;
    if (opl::same_phase16(input, output))
      return lease.launch_last(softmax_split_apply_kernel<T, true>, grid, dim3(kSplitThreads),
                               input, output, partials, cols, split.seg_len);
    return lease.launch_last(softmax_split_apply_kernel<T, false>, grid, dim3(kSplitThreads),
                             input, output, partials, cols, split.seg_len);
  }
  const bool vec =
      cols % E == 0 && opl::aligned16(input) && opl::aligned16(output);
  if (vec && cols <= 32 * E) {
    launch_group<T, E, 4>(opl::next_pow2(cols / E), input, output, rows, cols, stream);
    return hipGetLastError();
  }
  if (!vec && cols <= 32) {
    launch_group<T, 1, 8>(opl::next_pow2(cols), input, output, rows, cols, stream);
    return hipGetLastError();
  }
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
    case opl::RowPath::kTwoPass:  // split_plan takes every such row
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

extern "C" int operatorlib_softmax_f32(const float* input, float* output,
                                       int rows, int cols,
                                       void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  return softmax_launch(input, output, rows, cols, opl::ScratchSource{},
                        static_cast<hipStream_t>(stream_handle));
}

extern "C" int operatorlib_softmax_f16(const operatorlib_half_t* input,
                                       operatorlib_half_t* output, int rows,
                                       int cols, void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  return softmax_launch(reinterpret_cast<const _Float16*>(input),
                        reinterpret_cast<_Float16*>(output), rows, cols,
                        opl::ScratchSource{}, static_cast<hipStream_t>(stream_handle));
}

extern "C" size_t operatorlib_softmax_f32_workspace_size(int rows, int cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return split_bytes(rows, opl::split_plan(rows, cols));
}

extern "C" int operatorlib_softmax_f32_ws(const float* input, float* output, int rows,
                                          int cols, void* workspace, size_t workspace_bytes,
                                          void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  return softmax_launch(input, output, rows, cols,
                        opl::ScratchSource{true, workspace, workspace_bytes},
                        static_cast<hipStream_t>(stream_handle));
}

extern "C" size_t operatorlib_softmax_f16_workspace_size(int rows, int cols) {
  return operatorlib_softmax_f32_workspace_size(rows, cols);
}

extern "C" int operatorlib_softmax_f16_ws(const operatorlib_half_t* input,
                                          operatorlib_half_t* output, int rows, int cols,
                                          void* workspace, size_t workspace_bytes,
                                          void* stream_handle) {
  if (!opl::matrix_args_ok(input, output, rows, cols))
    return hipErrorInvalidValue;
  return softmax_launch(reinterpret_cast<const _Float16*>(input),
                        reinterpret_cast<_Float16*>(output), rows, cols,
                        opl::ScratchSource{true, workspace, workspace_bytes},
                        static_cast<hipStream_t>(stream_handle));
}
