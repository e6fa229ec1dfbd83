#pragma once
// Register-resident row slices for the row-wise bandwidth kernels (softmax,
// RMSNorm).
//
// A row is owned by a group of `Lanes` threads (one wavefront, or a whole
// workgroup for long rows). Thread t of the group holds the row's elements
//   W == 4:  float4 number  j * Lanes + t   (16-byte loads/stores; needs
//            cols % 4 == 0 and 16-byte aligned base pointers)
//   W == 1:  element        j * Lanes + t   (4-byte accesses; any shape)
// for j = 0 .. V-1. Consecutive lanes touch consecutive addresses, so every
// wave-wide access is one contiguous 256 B (W=1) or 1 KiB (W=4) segment.
// The whole row is read from HBM exactly once and written exactly once.
//
// Launch shapes (chosen by pick_row_plan):
//   cols <= 4096   one wavefront per row, 4 rows per 256-thread workgroup
//   cols <= 32768  one 512-thread workgroup per row
//   larger         two passes over HBM (row does not fit in registers)

#include <hip/hip_runtime.h>

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
