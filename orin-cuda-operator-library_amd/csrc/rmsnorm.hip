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
// Rows longer than 32768 columns, and a few long rows that would leave CUs
// idle, are cut into segments over workgroups and re-read x once.

#include <hip/hip_runtime.h>

#include <cstddef>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "rowwise.hpp"
#include "scratch.hpp"
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

// Short rows: a group of G lanes per row, 64 / G rows per wavefront, one
// access per lane (W = E: chunk t of aligned rows; W = 1: element t). A
// lane's weights are the same for every row it visits, so they are loaded
// once. A wavefront per row left most lanes idle here (1048576 x 16: 151 us
// against a 19.5 us copy of the same bytes).
template <typename T, int G, int W, int U>
__global__ __launch_bounds__(opl::kGroupThreads) void rmsnorm_group_kernel(
    const T* __restrict__ input, const T* __restrict__ weight,
    T* __restrict__ output, int rows, int cols, float epsilon) {
  using A = typename opl::Access<T, W>::type;
  constexpr int kRowsPerWave = opl::kWaveSize / G;
  constexpr int kWaves = opl::kGroupThreads / opl::kWaveSize;
  const int lane = threadIdx.x % opl::kWaveSize;
  const int t = lane % G;
  const int r_lane = lane / G;
  const bool lane_in = t * W < cols;
  const A wq = *reinterpret_cast<const A*>(weight + (lane_in ? t * W : 0));
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
      for (int e = 0; e < W; ++e) x[e] = in ? static_cast<float>(q[u][e]) : 0.0f;
      const float ss = opl::group_reduce<opl::SumOp, G>(sum_squares(x));
      const float inv = rsqrtf(ss / static_cast<float>(cols) + epsilon);
      if (in) {
        A y;
#pragma unroll
        for (int e = 0; e < W; ++e) y[e] = static_cast<T>((x[e] * inv) * static_cast<float>(wq[e]));
        __builtin_nontemporal_store(y, reinterpret_cast<A*>(output + row * cols + t * W));
      }
    }
  }
}

template <typename T, int W, int U, int G = 1>
void launch_group(int g, const T* in, const T* w, T* out, int rows, int cols, float eps,
                  hipStream_t stream) {
  if constexpr (G < 32) {
    if (g > G) return launch_group<T, W, U, 2 * G>(g, in, w, out, rows, cols, eps, stream);
  }
  constexpr int kRowsPerBlock = opl::kGroupThreads / G * U;
  const long long blocks = (static_cast<long long>(rows) + kRowsPerBlock - 1) / kRowsPerBlock;
  rmsnorm_group_kernel<T, G, W, U>
      <<<dim3(static_cast<unsigned>(blocks < opl::kGroupMaxBlocks ? blocks : opl::kGroupMaxBlocks)),
         dim3(opl::kGroupThreads), 0, stream>>>(in, w, out, rows, cols, eps);
}

// Rows over several workgroups (opl::split_plan: rows too long for
// registers, and few long rows; one workgroup per row took 1076 us for 4 x
// 2^20 and 42 us for 64 x 65536). Pass 1 writes every segment's sum of
// squares to scratch; pass 2 sums the row's partials in segment order
// (every wavefront of the row computes the same bits), re-reads its
// segment and writes (x * inv) * w.
using opl::kSplitThreads;
using opl::kSplitUnroll;
using opl::kSplitWaves;

template <typename T>
__global__ __launch_bounds__(kSplitThreads) void rmsnorm_split_stats_kernel(
    const T* __restrict__ input, float* __restrict__ partials, int cols, int seg_len) {
  using Chunk = typename opl::RowElem<T>::Chunk;
  constexpr int E = opl::RowElem<T>::kPerChunk;
  __shared__ float slots[kSplitWaves];
  const int c0 = blockIdx.y * seg_len;
  const int n = min(cols - c0, seg_len);
  const T* p = input + static_cast<std::size_t>(blockIdx.x) * cols + c0;
  const opl::Segment<T> sg(p, n);
  const Chunk* body = reinterpret_cast<const Chunk*>(p + sg.head);
  const int t = threadIdx.x;
  float ss = 0.0f;
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
        ss += sum_squares(x);
      }
    }
  }
  const int xc = sg.extra(t);
  if (xc >= 0) {
    const float x = static_cast<float>(p[xc]);
    ss += x * x;
  }
  ss = opl::block_reduce<opl::SumOp, kSplitWaves>(ss, slots);
  if (t == 0) partials[static_cast<std::size_t>(blockIdx.x) * gridDim.y + blockIdx.y] = ss;
}

// kChunks: input and output rows share their 16-byte phase (16-byte
// accesses on both sides; the weights as chunks too where their phase is
// the row's, else element by element from the caches); otherwise element
// accesses.
template <typename T, bool kChunks>
__global__ __launch_bounds__(kSplitThreads) void rmsnorm_split_apply_kernel(
    const T* __restrict__ input, const T* __restrict__ weight, T* __restrict__ output,
    const float* __restrict__ partials, int cols, int seg_len, float epsilon) {
  using Chunk = typename opl::RowElem<T>::Chunk;
  constexpr int E = opl::RowElem<T>::kPerChunk;
  const int segments = gridDim.y;
  const float* pr = partials + static_cast<std::size_t>(blockIdx.x) * segments;
  const int lane = threadIdx.x % opl::kWaveSize;
  float ps = 0.0f;
  for (int i = lane; i < segments; i += opl::kWaveSize) ps += pr[i];
  const float inv = rsqrtf(opl::wave_reduce<opl::SumOp>(ps) / static_cast<float>(cols) + epsilon);

  const int c0 = blockIdx.y * seg_len;
  const int n = min(cols - c0, seg_len);
  const std::size_t offset = static_cast<std::size_t>(blockIdx.x) * cols + c0;
  const T* p = input + offset;
  const T* w = weight + c0;
  T* o = output + offset;
  const int t = threadIdx.x;
  if constexpr (kChunks) {
    const opl::Segment<T> sg(p, n);
    const Chunk* body = reinterpret_cast<const Chunk*>(p + sg.head);
    Chunk* obody = reinterpret_cast<Chunk*>(o + sg.head);
    const T* wb = w + sg.head;
    const bool w_chunks = opl::aligned16(wb);  // uniform
    for (int i0 = t; i0 < sg.body; i0 += kSplitThreads * kSplitUnroll) {
      Chunk q[kSplitUnroll], wq[kSplitUnroll];
#pragma unroll
      for (int u = 0; u < kSplitUnroll; ++u) {
        const int i = i0 + u * kSplitThreads;
        const int ic = i < sg.body ? i : i0;
        q[u] = __builtin_nontemporal_load(body + ic);
        if (w_chunks) {
          wq[u] = reinterpret_cast<const Chunk*>(wb)[ic];
        } else {
#pragma unroll
          for (int e = 0; e < E; ++e) wq[u][e] = wb[E * ic + e];
        }
      }
#pragma unroll
      for (int u = 0; u < kSplitUnroll; ++u) {
        const int i = i0 + u * kSplitThreads;
        if (i < sg.body) {
          Chunk y;
#pragma unroll
          for (int e = 0; e < E; ++e)
            y[e] = static_cast<T>((static_cast<float>(q[u][e]) * inv) *
                                  static_cast<float>(wq[u][e]));
          __builtin_nontemporal_store(y, obody + i);
        }
      }
    }
    const int xc = sg.extra(t);
    if (xc >= 0)
      o[xc] = static_cast<T>((static_cast<float>(p[xc]) * inv) * static_cast<float>(w[xc]));
  } else {
    constexpr int U = 2 * kSplitUnroll;
    for (int i0 = t; i0 < n; i0 += kSplitThreads * U) {
      T q[U], wq[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kSplitThreads;
        const int ic = i < n ? i : i0;
        q[u] = __builtin_nontemporal_load(p + ic);
        wq[u] = w[ic];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = i0 + u * kSplitThreads;
        if (i < n)
          __builtin_nontemporal_store(
              static_cast<T>((static_cast<float>(q[u]) * inv) * static_cast<float>(wq[u])), o + i);
      }
    }
  }
}

inline std::size_t split_bytes(int rows, const opl::SplitPlan& p) {
  return p.segments > 0 ? sizeof(float) * static_cast<std::size_t>(rows) * p.segments : 0;
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
int rmsnorm_launch(const Args<T>& args, const opl::ScratchSource& src, hipStream_t stream) {
  constexpr int E = opl::RowElem<T>::kPerChunk;
  constexpr int kWaveMaxV = opl::kRowWaveMaxCols / (opl::kWaveSize * E);
  constexpr int kBlockMinV =
      2 * opl::kRowWaveMaxCols / (opl::kRowBlockThreads * E);
  constexpr int kBlockMaxV =
      opl::kRowBlockMaxCols / (opl::kRowBlockThreads * E);
  const int hidden = args.cols;
  const opl::SplitPlan split = opl::split_plan(args.rows, hidden);
  const std::size_t bytes = split_bytes(args.rows, split);
  if (src.workspace_mode && !opl::workspace_ok(src.data, src.bytes, bytes))
    return hipErrorInvalidValue;
  if (split.segments > 0) {
    // 4 bytes per (row, segment): fewer than 2 * kSplitTargetBlocks for
    // split rows, one per row otherwise; every plan fits the arena.
    opl::ScratchLease lease(stream, src.workspace_mode ? src.data : nullptr, src.bytes);
    if (lease.status() != hipSuccess) return lease.status();
    float* partials = static_cast<float*>(lease.data());
    // rows on x (up to 2^31 - 1), segments (at most 512) on y
    const dim3 grid(static_cast<unsigned>(args.rows), static_cast<unsigned>(split.segments));
    rmsnorm_split_stats_kernel<T><<<grid, dim3(kSplitThreads), 0, stream>>>(
        args.input, partials, hidden, split.seg_len);
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) return status;
    if (opl::same_phase16(args.input, args.output))
      return lease.launch_last(rmsnorm_split_apply_kernel<T, true>, grid, dim3(kSplitThreads),
                               args.input, args.weight, args.output, partials, hidden,
                               split.seg_len, args.epsilon);
    return lease.launch_last(rmsnorm_split_apply_kernel<T, false>, grid, dim3(kSplitThreads),
                             args.input, args.weight, args.output, partials, hidden,
                             split.seg_len, args.epsilon);
  }
  const bool vec = hidden % E == 0 && opl::aligned16(args.input) &&
                   opl::aligned16(args.weight) && opl::aligned16(args.output);
  if (vec && hidden <= 32 * E) {
    launch_group<T, E, 4>(opl::next_pow2(hidden / E), args.input, args.weight, args.output,
                          args.rows, hidden, args.epsilon, stream);
    return hipGetLastError();
  }
  if (!vec && hidden <= 32) {
    launch_group<T, 1, 8>(opl::next_pow2(hidden), args.input, args.weight, args.output,
                          args.rows, hidden, args.epsilon, stream);
    return hipGetLastError();
  }
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
    case opl::RowPath::kTwoPass:  // opl::split_plan takes every such row
      return hipErrorInvalidValue;
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
      Args<float>{input, weight, output, tokens, hidden, epsilon}, opl::ScratchSource{},
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
      opl::ScratchSource{}, static_cast<hipStream_t>(stream_handle));
}

extern "C" size_t operatorlib_rmsnorm_f32_workspace_size(int tokens, int hidden) {
  if (tokens <= 0 || hidden <= 0) return 0;
  return split_bytes(tokens, opl::split_plan(tokens, hidden));
}

extern "C" int operatorlib_rmsnorm_f32_ws(const float* input, const float* weight,
                                          float* output, int tokens, int hidden,
                                          float epsilon, void* workspace,
                                          size_t workspace_bytes, void* stream_handle) {
  if (!opl::rmsnorm_args_ok(input, weight, output, tokens, hidden, epsilon))
    return hipErrorInvalidValue;
  return rmsnorm_launch(Args<float>{input, weight, output, tokens, hidden, epsilon},
                        opl::ScratchSource{true, workspace, workspace_bytes},
                        static_cast<hipStream_t>(stream_handle));
}

extern "C" size_t operatorlib_rmsnorm_f16_workspace_size(int tokens, int hidden) {
  return operatorlib_rmsnorm_f32_workspace_size(tokens, hidden);
}

extern "C" int operatorlib_rmsnorm_f16_ws(const operatorlib_half_t* input,
                                          const operatorlib_half_t* weight,
                                          operatorlib_half_t* output, int tokens, int hidden,
                                          float epsilon, void* workspace,
                                          size_t workspace_bytes, void* stream_handle) {
  if (!opl::rmsnorm_args_ok(input, weight, output, tokens, hidden, epsilon))
    return hipErrorInvalidValue;
  return rmsnorm_launch(
      Args<_Float16>{reinterpret_cast<const _Float16*>(input),
                     reinterpret_cast<const _Float16*>(weight),
                     reinterpret_cast<_Float16*>(output), tokens, hidden, epsilon},
      opl::ScratchSource{true, workspace, workspace_bytes},
      static_cast<hipStream_t>(stream_handle));
}
