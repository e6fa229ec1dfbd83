#pragma once
// Register-resident row slices for the row-wise bandwidth kernels (softmax,
// RMSNorm).
//
// A row is owned by a group of `Lanes` threads (one wavefront, or a whole
// workgroup for long rows). Thread t of the group holds the row's elements
//   W == 4:  float4 number  j * Lanes + t   (16-byte loads/stores; needs
//            cols % 4 == 0 and 16-byte aligned base pointers)
//   W == 1:  element        j * Lanes + t   (4-byte accesses; any shape)
// for j = 0 .. V-1; RaggedRowSlice (below) keeps 16-byte accesses for rows
// of any length and alignment. Consecutive lanes touch consecutive addresses, so every
// wave-wide access is one contiguous 256 B (W=1) or 1 KiB (W=4) segment.
// The whole row is read from HBM exactly once and written exactly once.
//
// Launch shapes (chosen by pick_row_plan):
//   cols <= 4096   one wavefront per row, 4 rows per 256-thread workgroup
//   cols <= 32768  one 512-thread workgroup per row
//   larger         two passes over HBM (row does not fit in registers)

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace opl {

constexpr int kRowWaveThreads = 256;  // 4 wavefronts, one row each
constexpr int kRowWaveRows = kRowWaveThreads / kWaveSize;
constexpr int kRowBlockThreads = 512; // one row per workgroup
constexpr int kRowBlockWaves = kRowBlockThreads / kWaveSize;
constexpr int kRowWaveMaxCols = 4096;
constexpr int kRowBlockMaxCols = 32768;

template <int V, int Lanes, int W>
struct RowSlice {
  static constexpr int kCount = V * W;
  float x[kCount];

  __device__ __forceinline__ static int first_col(int t, int j) {
    return (j * Lanes + t) * W;
  }

  __device__ __forceinline__ void load(const float* __restrict__ row,
                                       int cols, int t, float pad) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int c = first_col(t, j);
      if constexpr (W == 4) {
        float4 q = make_float4(pad, pad, pad, pad);
        if (c < cols) q = *reinterpret_cast<const float4*>(row + c);
        x[4 * j + 0] = q.x;
        x[4 * j + 1] = q.y;
        x[4 * j + 2] = q.z;
        x[4 * j + 3] = q.w;
      } else {
        x[j] = c < cols ? row[c] : pad;
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ row, int cols,
                                        int t) const {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int c = first_col(t, j);
      if (c < cols) {
        if constexpr (W == 4) {
          *reinterpret_cast<float4*>(row + c) =
              make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
        } else {
          row[c] = x[j];
        }
      }
    }
  }

  // True when register slot i holds a real element of the row.
  __device__ __forceinline__ static bool valid(int t, int i, int cols) {
    return first_col(t, i / W) + (i % W) < cols;
  }
};

// A row at any 4-byte alignment and of any length, still moved with
// 16-byte accesses: a scalar head (the 0-3 elements before the row's first
// 16-byte boundary), an aligned float4 body, and a scalar tail (< 4
// elements). Thread t holds body float4s j * Lanes + t (j < V) in x[0, 4V)
// and at most one head or tail element in x[4V]: threads 0-2 the head,
// threads 4-6 the tail. Input and output rows must share their offset
// modulo 16 bytes (the layout is computed once from the input row), and
// rows must hold at least kRaggedMinCols elements, so the body is never
// empty.
constexpr int kRaggedMinCols = 8;

template <int V, int Lanes>
struct RaggedRowSlice {
  static constexpr int kCount = 4 * V + 1;
  float x[kCount];
  int head;        // elements before the first 16-byte boundary
  int body;        // float4s in the aligned body
  int tail_start;  // first tail element (head + 4 * body)

  __device__ __forceinline__ void layout(const float* row, int cols) {
    head = static_cast<int>(((16 - (reinterpret_cast<uintptr_t>(row) & 15)) & 15) >> 2);
    if (head > cols) head = cols;
    body = (cols - head) >> 2;
    tail_start = head + 4 * body;
  }

  // Column held in x[4V] by thread t, or -1.
  __device__ __forceinline__ int extra_col(int t, int cols) const {
    if (t < head) return t;
    const int c = tail_start + t - 4;
    return (t >= 4 && c < cols) ? c : -1;
  }

  // Column of body slot i (0 <= i < 4V) of thread t; valid if < tail_start.
  __device__ __forceinline__ int body_col(int t, int i) const {
    return head + 4 * ((i / 4) * Lanes + t) + (i % 4);
  }

  // Loads are unconditional (indices clamped into the row), so they issue
  // back to back without per-load branches: load_raw() only issues them,
  // mask() later replaces the out-of-range slots by `pad` (which waits for
  // the data), and load() does both.
  __device__ __forceinline__ void load_raw(const float* __restrict__ row,
                                           int cols, int t) {
    layout(row, cols);
    const float4* b4 = reinterpret_cast<const float4*>(row + head);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int q = j * Lanes + t;
      const float4 v = b4[q < body ? q : body - 1];
      x[4 * j + 0] = v.x;
      x[4 * j + 1] = v.y;
      x[4 * j + 2] = v.z;
      x[4 * j + 3] = v.w;
    }
    const int c = extra_col(t, cols);
    x[4 * V] = row[c >= 0 ? c : 0];
  }

  __device__ __forceinline__ void mask(int cols, int t, float pad) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const bool in = j * Lanes + t < body;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * j + e] = in ? x[4 * j + e] : pad;
    }
    x[4 * V] = extra_col(t, cols) >= 0 ? x[4 * V] : pad;
  }

  __device__ __forceinline__ void load(const float* __restrict__ row,
                                       int cols, int t, float pad) {
    load_raw(row, cols, t);
    mask(cols, t, pad);
  }

  __device__ __forceinline__ void store(float* __restrict__ row, int cols,
                                        int t) const {
    float4* b4 = reinterpret_cast<float4*>(row + head);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int q = j * Lanes + t;
      if (q < body)
        b4[q] = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
    }
    const int c = extra_col(t, cols);
    if (c >= 0) row[c] = x[4 * V];
  }
};

// Slice type for an access width: 4 -> aligned float4 rows, 1 -> 4-byte
// elements, 0 -> ragged rows (float4 body at any alignment).
template <int V, int Lanes, int W>
struct SliceFor {
  using type = RowSlice<V, Lanes, W>;
};
template <int V, int Lanes>
struct SliceFor<V, Lanes, 0> {
  using type = RaggedRowSlice<V, Lanes>;
};

// Same offset modulo 16 bytes.
inline bool same_phase16(const void* a, const void* b) {
  return ((reinterpret_cast<uintptr_t>(a) ^ reinterpret_cast<uintptr_t>(b)) & 15) == 0;
}

enum class RowPath { kWave, kBlock, kTwoPass };

struct RowPlan {
  RowPath path;
  int vec_width;   // W: 4 or 1
  int per_thread;  // V: accesses per thread (power of two)
};

inline int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

inline RowPlan pick_row_plan(int cols, bool vec4_ok) {
  const int w = vec4_ok ? 4 : 1;
  if (cols <= kRowWaveMaxCols)
    return {RowPath::kWave, w, next_pow2((cols + kWaveSize * w - 1) /
                                         (kWaveSize * w))};
  if (cols <= kRowBlockMaxCols)
    return {RowPath::kBlock, w,
            next_pow2((cols + kRowBlockThreads * w - 1) /
                      (kRowBlockThreads * w))};
  return {RowPath::kTwoPass, w, 0};
}

}  // namespace opl
