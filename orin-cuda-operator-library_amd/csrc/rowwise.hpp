#pragma once
// Register-resident row slices for the row-wise bandwidth kernels (softmax,
// RMSNorm).
//
// A row is owned by a group of `Lanes` threads (one wavefront, or a whole
// workgroup for long rows). Rows are stored as fp32 or fp16 (T) and held
// in VGPRs as fp32. Thread t of the group holds the row's elements
//   W == E:  16-byte chunk  j * Lanes + t   (E = 4 fp32 or 8 fp16 elements;
//            needs cols % E == 0 and 16-byte aligned base pointers)
//   W == 1:  element        j * Lanes + t   (any shape)
// for j = 0 .. V-1; RaggedRowSlice (below) keeps 16-byte accesses for rows
// of any length and alignment. Consecutive lanes touch consecutive
// addresses, so every wave-wide access is one contiguous segment (1 KiB for
// 16-byte chunks). The whole row is read from HBM exactly once and written
// exactly once.
//
// Launch shapes:
//   short rows     groups of G <= 32 lanes per row (up to 32 elements, or
//                  32 chunks of aligned rows; group_reduce)
//   cols <= 4096   one wavefront per row, 4 rows per 256-thread workgroup
//   cols <= 32768  one 512-thread workgroup per row (pick_row_plan)
//   longer rows,   segments over workgroups, two passes over HBM
//   few long rows  (split_plan, Segment)

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

// Storage formats of a row. Rows are kept in VGPRs as fp32 whatever the
// storage type; Chunk is one 16-byte access (4 fp32 or 8 fp16 elements).
template <typename T>
struct RowElem;
template <>
struct RowElem<float> {
  typedef float Chunk __attribute__((ext_vector_type(4)));
  static constexpr int kPerChunk = 4;
};
template <>
struct RowElem<_Float16> {
  typedef _Float16 Chunk __attribute__((ext_vector_type(8)));
  static constexpr int kPerChunk = 8;
};

template <int V, int Lanes, int W, typename T = float>
struct RowSlice {
  using Chunk = typename RowElem<T>::Chunk;
  static_assert(W == 1 || W == RowElem<T>::kPerChunk, "access width");
  static constexpr int kCount = V * W;
  float x[kCount];

  __device__ __forceinline__ static int first_col(int t, int j) {
    return (j * Lanes + t) * W;
  }

  // Every load is issued from a clamped index (element / chunk 0 always
  // exists: cols >= W), and out-of-row slots are replaced afterwards. A
  // load inside a per-slot branch makes the compiler wait for it inside the
  // branch (s_waitcnt vmcnt(0) per slot), serialising the row's loads.
  // kStream = true issues non-temporal loads (rows read once; the
  // weights of RMSNorm, re-read by every row, use the default).
  template <bool kStream = false>
  __device__ __forceinline__ void load(const T* __restrict__ row, int cols,
                                       int t, float pad) {
    if constexpr (W > 1) {
      Chunk q[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int c = first_col(t, j);
        const Chunk* src = reinterpret_cast<const Chunk*>(row + (c < cols ? c : 0));
        q[j] = kStream ? __builtin_nontemporal_load(src) : *src;
      }
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const bool in = first_col(t, j) < cols;
#pragma unroll
        for (int e = 0; e < W; ++e)
          x[W * j + e] = in ? static_cast<float>(q[j][e]) : pad;
      }
    } else {
      T q[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int c = first_col(t, j);
        const T* src = row + (c < cols ? c : 0);
        q[j] = kStream ? __builtin_nontemporal_load(src) : *src;
      }
#pragma unroll
      for (int j = 0; j < V; ++j)
        x[j] = first_col(t, j) < cols ? static_cast<float>(q[j]) : pad;
    }
  }

  // Non-temporal stores (outputs are never re-read by the kernel). Cached
  // stores left the caches full of dirty output lines, which cost the next
  // kernel on the stream: softmax 4096 x 1024 followed by RMSNorm 2048 x
  // 4096, inputs cycling through 1 GiB, measured 24.9 us per pair with
  // cached loads and stores, 18.6 us with non-temporal stores and 18.1 us
  // with non-temporal loads as well.
  __device__ __forceinline__ void store(T* __restrict__ row, int cols,
                                        int t) const {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int c = first_col(t, j);
      if (c < cols) {
        if constexpr (W > 1) {
          Chunk q;
#pragma unroll
          for (int e = 0; e < W; ++e) q[e] = static_cast<T>(x[W * j + e]);
          __builtin_nontemporal_store(q, reinterpret_cast<Chunk*>(row + c));
        } else {
          __builtin_nontemporal_store(static_cast<T>(x[j]), row + c);
        }
      }
    }
  }

  // True when register slot i holds a real element of the row.
  __device__ __forceinline__ static bool valid(int t, int i, int cols) {
    return first_col(t, i / W) + (i % W) < cols;
  }
};

// A row at any element alignment and of any length, still moved with
// 16-byte accesses: a scalar head (the 0 to E-1 elements before the row's
// first 16-byte boundary, E elements per chunk), an aligned chunk body, and
// a scalar tail (< E elements). Thread t holds body chunks j * Lanes + t
// (j < V) in x[0, E*V) and at most one head or tail element in x[E*V]:
// threads 0 .. E-2 the head, threads E .. 2E-2 the tail. Input and output
// rows must share their offset modulo 16 bytes (the layout is computed once
// from the input row), and rows must hold at least kMinCols = 2E elements,
// so the body is never empty.
template <int V, int Lanes, typename T = float>
struct RaggedRowSlice {
  using Chunk = typename RowElem<T>::Chunk;
  static constexpr int kE = RowElem<T>::kPerChunk;
  static_assert(kE == 4 || kE == 8, "chunk of 4 or 8 elements");
  static constexpr int kMinCols = 2 * kE;
  static_assert(Lanes >= 2 * kE, "head and tail need 2E lanes");
  static constexpr int kCount = kE * V + 1;
  float x[kCount];
  int head;        // elements before the first 16-byte boundary
  int body;        // chunks in the aligned body
  int tail_start;  // first tail element (head + E * body)

  __device__ __forceinline__ void layout(const T* row, int cols) {
    head = static_cast<int>(((16 - (reinterpret_cast<uintptr_t>(row) & 15)) & 15) /
                            sizeof(T));
    if (head > cols) head = cols;
    body = (cols - head) >> (kE == 8 ? 3 : 2);  // cols - head >= 0
    tail_start = head + kE * body;
  }

  // Column held in x[E*V] by thread t, or -1.
  __device__ __forceinline__ int extra_col(int t, int cols) const {
    if (t < head) return t;
    const int c = tail_start + t - kE;
    return (t >= kE && c < cols) ? c : -1;
  }

  // Column of body slot i (0 <= i < E*V) of thread t; valid if < tail_start.
  __device__ __forceinline__ int body_col(int t, int i) const {
    return head + kE * ((i / kE) * Lanes + t) + (i % kE);
  }

  // Loads are unconditional (indices clamped into the row), so they issue
  // back to back without per-load branches: load_raw() only issues them,
  // mask() later replaces the out-of-range slots by `pad` (which waits for
  // the data), and load() does both. kStream as in RowSlice::load.
  template <bool kStream = false>
  __device__ __forceinline__ void load_raw(const T* __restrict__ row,
                                           int cols, int t) {
    layout(row, cols);
    const Chunk* b = reinterpret_cast<const Chunk*>(row + head);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int q = j * Lanes + t;
      const Chunk* src = b + (q < body ? q : body - 1);
      const Chunk v = kStream ? __builtin_nontemporal_load(src) : *src;
#pragma unroll
      for (int e = 0; e < kE; ++e) x[kE * j + e] = static_cast<float>(v[e]);
    }
    const int c = extra_col(t, cols);
    x[kE * V] = static_cast<float>(row[c >= 0 ? c : 0]);
  }

  __device__ __forceinline__ void mask(int cols, int t, float pad) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const bool in = j * Lanes + t < body;
#pragma unroll
      for (int e = 0; e < kE; ++e) x[kE * j + e] = in ? x[kE * j + e] : pad;
    }
    x[kE * V] = extra_col(t, cols) >= 0 ? x[kE * V] : pad;
  }

  template <bool kStream = false>
  __device__ __forceinline__ void load(const T* __restrict__ row, int cols,
                                       int t, float pad) {
    load_raw<kStream>(row, cols, t);
    mask(cols, t, pad);
  }

  // Non-temporal stores, as in RowSlice::store.
  __device__ __forceinline__ void store(T* __restrict__ row, int cols,
                                        int t) const {
    Chunk* b = reinterpret_cast<Chunk*>(row + head);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int q = j * Lanes + t;
      if (q < body) {
        Chunk v;
#pragma unroll
        for (int e = 0; e < kE; ++e) v[e] = static_cast<T>(x[kE * j + e]);
        __builtin_nontemporal_store(v, b + q);
      }
    }
    const int c = extra_col(t, cols);
    if (c >= 0) __builtin_nontemporal_store(static_cast<T>(x[kE * V]), row + c);
  }
};

// Slice type for an access width: RowElem<T>::kPerChunk -> aligned 16-byte
// chunks, 1 -> single elements, 0 -> ragged rows (chunk body at any
// alignment).
template <int V, int Lanes, int W, typename T = float>
struct SliceFor {
  using type = RowSlice<V, Lanes, W, T>;
};
template <int V, int Lanes, typename T>
struct SliceFor<V, Lanes, 0, T> {
  using type = RaggedRowSlice<V, Lanes, T>;
};

// Short-row kernels: groups of G lanes per row, one access of W elements
// per lane (W = E: a 16-byte chunk, W = 1: one element), workgroups of
// kGroupThreads striding over blocks of rows.
constexpr int kGroupThreads = 256;
constexpr int kGroupMaxBlocks = 2048;

template <typename T, int W>
struct Access {
  using type = typename RowElem<T>::Chunk;
};
template <typename T>
struct Access<T, 1> {
  typedef T type __attribute__((ext_vector_type(1)));
};

// All-reduce over aligned groups of G lanes of a wavefront (G = 1, 2, 4, 8,
// 16 or 32): every lane of a group receives the group's value. These are
// wave_reduce's first log2(G) butterfly steps, so the bits are the same in
// every lane of a group; all 64 lanes must be active.
template <class Op, int G>
__device__ __forceinline__ float group_reduce(float v) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32, "group size");
  if constexpr (G >= 2) v = Op::apply(v, dpp_f32<kDppQuadXor1>(v));
  if constexpr (G >= 4) v = Op::apply(v, dpp_f32<kDppQuadXor2>(v));
  if constexpr (G >= 8) v = Op::apply(v, dpp_f32<kDppRowHalfMirror>(v));
  if constexpr (G >= 16) v = Op::apply(v, dpp_f32<kDppRowMirror>(v));
  if constexpr (G >= 32) v = combine_xor16_f32<Op>(v);
  return v;
}

// n elements from p (a segment of a row, at any element alignment) walked
// with 16-byte accesses: `head` elements up to the first 16-byte boundary,
// `body` aligned chunks of E elements, then `tail` (< E) elements.
template <typename T>
struct Segment {
  static constexpr int kE = RowElem<T>::kPerChunk;
  int head, body, tail;
  __device__ __forceinline__ Segment(const T* p, int n) {
    head = static_cast<int>(((16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15) / sizeof(T));
    if (head > n) head = n;
    body = (n - head) / kE;
    tail = n - head - kE * body;
  }
  // The element outside the body that thread t handles, or -1: threads
  // 0 .. head-1 the head, threads E .. E+tail-1 the tail.
  __device__ __forceinline__ int extra(int t) const {
    if (t < head) return t;
    if (t >= kE && t - kE < tail) return head + kE * body + (t - kE);
    return -1;
  }
};

// Rows over several workgroups (softmax, RMSNorm): a row is cut into
// `segments` segments of seg_len elements, one kSplitThreads workgroup
// each; pass 1 writes a per-segment partial to scratch, pass 2 combines the
// row's partials in segment order and re-reads its segment. Every row
// longer than kRowBlockMaxCols (too long for registers) takes this path,
// in as many segments as fill kSplitTargetBlocks workgroups (one when there
// are that many rows); register-resident rows of a workgroup (kRowWaveMaxCols
// < cols <= kRowBlockMaxCols) only when there are fewer than kSplitMaxRows
// of them, which would leave most CUs idle.
constexpr int kSplitThreads = 256;
constexpr int kSplitWaves = kSplitThreads / kWaveSize;
constexpr int kSplitUnroll = 4;          // 16-byte chunks in flight per thread
constexpr int kSplitTargetBlocks = 512;  // two workgroups per CU of a 256-CU MI355X
constexpr int kSplitMinSegment = 2048;   // elements
constexpr int kSplitMaxRows = 64;

struct SplitPlan {
  int segments = 0;  // 0: not split
  int seg_len = 0;   // elements, a multiple of 64
};

inline SplitPlan split_plan(int rows, int cols) {
  SplitPlan p;
  if (cols <= kRowWaveMaxCols) return p;
  const bool long_rows = cols > kRowBlockMaxCols;
  if (!long_rows && rows >= kSplitMaxRows) return p;
  const int by_rows =
      static_cast<int>((static_cast<long long>(kSplitTargetBlocks) + rows - 1) / rows);
  const int by_cols = cols / kSplitMinSegment;
  const int want = by_rows < by_cols ? by_rows : by_cols;
  if (want < (long_rows ? 1 : 2)) return p;
  const int per = (cols + want - 1) / want;
  p.seg_len = (per + 63) / 64 * 64;
  p.segments = (cols + p.seg_len - 1) / p.seg_len;
  return p;
}

// Same offset modulo 16 bytes.
inline bool same_phase16(const void* a, const void* b) {
  return ((reinterpret_cast<uintptr_t>(a) ^ reinterpret_cast<uintptr_t>(b)) & 15) == 0;
}

enum class RowPath { kWave, kBlock, kTwoPass };

struct RowPlan {
  RowPath path;
  int vec_width;   // W: elements per access (1, 4 or 8)
  int per_thread;  // V: accesses per thread (power of two)
};

inline int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

inline RowPlan pick_row_plan(int cols, int w) {
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
