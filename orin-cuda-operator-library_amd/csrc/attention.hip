// FlashAttention-style forward on the CDNA4 matrix cores.
//   attention_f16: fp16 Q/K/V, v_mfma_f32_16x16x32_f16 (fast path) or
//                  32x32x16, fp32 scores and online-softmax state, P rounded
//                  to fp16 for P.V, fp32 out
//   attention_f32: fp32 Q/K/V, v_mfma_f32_32x32x2_f32, all fp32
//
// Reference: operatorlib::attention_f16 / attention_f32
// (src/attention.cu:445-507). Same maths: per (batch, head),
//   O = softmax(Q K^T / sqrt(D), keys j > row i hidden when causal) V,
// computed with the online recurrence m' = max(m, x), a = e^(m - m'),
// l' = a l + sum e^(x - m'), O' = a O + e^(x - m') V (src/attention.cu:116-134,
// :296-349) so no S x S matrix is ever stored. As in the reference FP16
// path, P is rounded to fp16 before the P.V product; the reference's row
// sum adds the unrounded fp32 values (src/attention.cu:313-320), as does
// attention_mfma_kernel, while the fp16 fast path adds the rounded ones on
// the matrix cores (a relative difference of at most 2^-11 per term).
//
// Two kernels share the design below: attention_f16_dma_kernel (fp16,
// head_dim 64/128, any S, aligned tensors; described before it) and
// attention_mfma_kernel (every other shape and fp32), which stages K / V
// through registers.
//
// MI355X design, per 256-thread workgroup (4 wavefronts x 32 query rows;
// the register-staged kernel's lane layout, the fp16 fast path's is
// described before it):
//   * scores are computed transposed, S^T = K Q^T, so lane l of a wavefront
//     owns query row (l % 32): its row max / row sum need only the lane's
//     own registers plus one exchange with lane l ^ 32;
//   * the S^T accumulator registers are exactly the B operand of the next
//     MFMA, O^T += V^T P^T, so P never leaves registers; V is stored
//     transposed in LDS with its keys permuted to match that register
//     layout (fp16), or read row-wise straight from LDS (fp32);
//   * K / V tiles (64 keys fp16, 32 keys fp32) are double-buffered in LDS;
//     global loads of tile t+1 overlap the MFMAs of tile t;
//   * exp is exp2 on v_exp_f32 with log2(e)/sqrt(D) folded into one FMA;
//     the O rescale is skipped when no row max in the wavefront moved;
//   * causal: key tiles beyond the workgroup's last row are never loaded,
//     wavefronts skip tiles beyond their own rows, masks are applied only on
//     diagonal / ragged tiles; workgroups are issued heaviest-first, and
//     all workgroups of one head share an XCD (and its L2);
//   * grids too small to fill the GPU split each query block's keys: the
//     fp16 fast path between two or four wavefront groups of one workgroup
//     (merged through LDS), the register-staged kernel over several workgroups
//     (partials in scratch, the GPU's arena or the caller's workspace, merged by
//     attention_combine_kernel in split order).
// Head dims are padded to a multiple of 32 with zeros (any 1 <= D <= 128).

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "scratch.hpp"
#include "validate.hpp"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / opl::kWaveSize;
constexpr int kRowsPerWave = 32;
constexpr int kBlockRows = kWaves * kRowsPerWave;  // 128

template <typename T>
struct AttnPrec;

template <>
struct AttnPrec<_Float16> {
  using Chunk = half8;                // 16 bytes of Q / K / V
  static constexpr int kKeyTiles = 2;  // 32-key MFMA tiles per K/V tile
  __device__ __forceinline__ static void mma(floatx16& acc, const Chunk& a,
                                             const Chunk& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
  }
};

template <>
struct AttnPrec<float> {
  using Chunk = float4v;
  static constexpr int kKeyTiles = 1;
  __device__ __forceinline__ static void mma(floatx16& acc, const Chunk& a,
                                             const Chunk& b) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);
  }
};

template <typename T, int NDT>
struct AttnLayout {
  static constexpr int E = 16 / sizeof(T);          // elements per chunk
  static constexpr int kDP = 32 * NDT;              // padded head dim
  static constexpr int kKeys = 32 * AttnPrec<T>::kKeyTiles;  // keys per tile
  static constexpr int kDChunks = kDP / E;          // chunks per K/V row
  static constexpr int kChunkPairs = kDChunks / 2;  // MFMA k-steps over d
  // K tile: [kKeys][kDP], row pitch padded by 16 B.
  static constexpr int kKPitch = kDP * sizeof(T) + 16;
  static constexpr int kKBytes = kKeys * kKPitch;
  // V tile: fp16 -> transposed [kDP][kKeys] (keys permuted), pitch + 16 B;
  //         fp32 -> row-major [kKeys][kDP + 8] (rows r and r+4 land 32
  //         banks apart for the column reads).
  static constexpr int kVPitch = sizeof(T) == 2 ? kKeys * 2 + 16
                                                : (kDP + 8) * 4;
  static constexpr int kVBytes = sizeof(T) == 2 ? kDP * kVPitch
                                                : kKeys * kVPitch;
  static constexpr int kStageBytes = kKBytes + kVBytes;
  static constexpr int kLdsBytes = 2 * kStageBytes;
};

// Position of key r (0..15) inside its 16-key group of the transposed fp16
// V tile: the two middle quads swap, so that lane half h finds the 8 keys
// of its P^T operand (keys 4h..4h+3 and 8+4h..8+4h+3) contiguous.
__device__ __forceinline__ int vt_pos(int r) {
  return 8 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3);
}

template <typename T, bool kVector>
__device__ __forceinline__ typename AttnPrec<T>::Chunk load_chunk(
    const T* base, int row, int rows, int col, int cols, int ld) {
  using Chunk = typename AttnPrec<T>::Chunk;
  constexpr int E = 16 / sizeof(T);
  Chunk v;
  if constexpr (kVector) {
    if (row < rows && col < cols) {
      v = *reinterpret_cast<const Chunk*>(
          base + static_cast<std::size_t>(row) * ld + col);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = T(0);
    }
  } else {
    const T* p = base + static_cast<std::size_t>(row) * ld;
#pragma unroll
    for (int e = 0; e < E; ++e)
      v[e] = (row < rows && col + e < cols) ? p[col + e] : T(0);
  }
  return v;
}

// Global -> register staging of one K/V tile, then register -> LDS.
template <typename T, int NDT, bool kVector>
struct KvStager {
  using L = AttnLayout<T, NDT>;
  using Chunk = typename AttnPrec<T>::Chunk;
  static constexpr int E = L::E;
  static constexpr int kKItems = L::kKeys * L::kDChunks;             // chunks
  static constexpr int kKPerThread = (kKItems + kThreads - 1) / kThreads;
  // fp16 V: E x E blocks (E keys x E dims); fp32 V: plain chunks like K.
  static constexpr int kVItems =
      sizeof(T) == 2 ? (L::kKeys / E) * (L::kDP / E) : kKItems;
  static constexpr int kVPerThread = (kVItems + kThreads - 1) / kThreads;
  static constexpr int kVRows = sizeof(T) == 2 ? E : 1;

  Chunk k[kKPerThread];
  Chunk v[kVPerThread][kVRows];

  __device__ __forceinline__ void load(const T* kbase, const T* vbase,
                                       int key0, int S, int D) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kKPerThread; ++i) {
      const int q = tid + kThreads * i;
      if (q < kKItems) {
        const int key = q / L::kDChunks;
        const int c = q % L::kDChunks;
        k[i] = load_chunk<T, kVector>(kbase, key0 + key, S, c * E, D, D);
      }
    }
#pragma unroll
    for (int i = 0; i < kVPerThread; ++i) {
      const int q = tid + kThreads * i;
      if (q < kVItems) {
        if constexpr (sizeof(T) == 2) {
          const int kb = q / (L::kDP / E);  // key block of E keys
          const int c = q % (L::kDP / E);   // dim chunk
#pragma unroll
          for (int r = 0; r < E; ++r)
            v[i][r] = load_chunk<T, kVector>(vbase, key0 + kb * E + r, S,
                                             c * E, D, D);
        } else {
          const int key = q / L::kDChunks;
          const int c = q % L::kDChunks;
          v[i][0] = load_chunk<T, kVector>(vbase, key0 + key, S, c * E, D, D);
        }
      }
    }
  }

  __device__ __forceinline__ void store(unsigned char* stage) const {
    const int tid = threadIdx.x;
    unsigned char* sk = stage;
    unsigned char* sv = stage + L::kKBytes;
#pragma unroll
    for (int i = 0; i < kKPerThread; ++i) {
      const int q = tid + kThreads * i;
      if (q < kKItems) {
        const int key = q / L::kDChunks;
        const int c = q % L::kDChunks;
        *reinterpret_cast<Chunk*>(sk + key * L::kKPitch + c * 16) = k[i];
      }
    }
#pragma unroll
    for (int i = 0; i < kVPerThread; ++i) {
      const int q = tid + kThreads * i;
      if (q < kVItems) {
        if constexpr (sizeof(T) == 2) {
          const int kb = q / (L::kDP / E);
          const int c = q % (L::kDP / E);
          // Keys kb*8 .. kb*8+7 sit in 16-key group kb/2 at positions
          // vt_pos(8*(kb%2) + r): two runs of 4 contiguous keys.
          const int group_byte = (kb >> 1) * 32;
          const int p0 = vt_pos(8 * (kb & 1)) * 2;
          const int p1 = vt_pos(8 * (kb & 1) + 4) * 2;
#pragma unroll
          for (int dd = 0; dd < E; ++dd) {
            half4 lo, hi;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              lo[r] = v[i][r][dd];
              hi[r] = v[i][r + 4][dd];
            }
            unsigned char* row = sv + (c * E + dd) * L::kVPitch + group_byte;
            *reinterpret_cast<half4*>(row + p0) = lo;
            *reinterpret_cast<half4*>(row + p1) = hi;
          }
        } else {
          const int key = q / L::kDChunks;
          const int c = q % L::kDChunks;
          *reinterpret_cast<Chunk*>(sv + key * L::kVPitch + c * 16) = v[i][0];
        }
      }
    }
  }
};

template <typename T, int NDT, bool kVector, bool kSplit>
__global__ __launch_bounds__(kThreads) void attention_mfma_kernel(
    const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
    float* __restrict__ O, int BH, int S, int D, int causal,
    float score_scale_log2, int splits, float* __restrict__ part_o,
    float* __restrict__ part_ml) {
  using L = AttnLayout<T, NDT>;
  using Pr = AttnPrec<T>;
  using Chunk = typename Pr::Chunk;
  constexpr int NKB = Pr::kKeyTiles;
  __shared__ __attribute__((aligned(16))) unsigned char lds[L::kLdsBytes];

  // Heaviest query blocks first; all blocks of one head map to one XCD
  // (launch index modulo 8) whenever BH is a multiple of 8.
  // With splits > 1 (small grids) the key tiles of a query block are dealt
  // to `splits` workgroups; each writes its unnormalised O, row max and row
  // sum to part_o / part_ml and attention_combine_kernel merges them.
  const int q_blocks = (S + kBlockRows - 1) / kBlockRows;
  const unsigned item = kSplit ? blockIdx.x / splits : blockIdx.x;
  const int split = kSplit ? static_cast<int>(blockIdx.x % splits) : 0;
  const int qb = q_blocks - 1 - static_cast<int>(item / BH);
  const int bh = static_cast<int>(item % BH);
  const int q0 = qb * kBlockRows;

  const int lane = threadIdx.x % opl::kWaveSize;
  const int wave = threadIdx.x / opl::kWaveSize;
  const int half = lane / 32;
  const int l32 = lane % 32;
  const int wave_row0 = q0 + wave * kRowsPerWave;
  const int my_row = wave_row0 + l32;

  const std::size_t head = static_cast<std::size_t>(bh) * S * D;
  const T* qh = Q + head;
  const T* kh = K + head;
  const T* vh = V + head;

  // Q^T operand: lane (row, half) holds chunk (2c + half) of its row.
  Chunk qf[L::kChunkPairs];
#pragma unroll
  for (int c = 0; c < L::kChunkPairs; ++c)
    qf[c] = load_chunk<T, kVector>(qh, my_row, S, (2 * c + half) * L::E, D, D);

  floatx16 o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;
  float row_max = -FLT_MAX;  // finite sentinel: e^(sentinel - m) == 0
  float row_sum = 0.0f;      // this lane's half of the row sum

  const int visible_end = causal ? min(S, q0 + kBlockRows) : S;
  const int all_tiles = (visible_end + L::kKeys - 1) / L::kKeys;
  // This workgroup's tiles: [tile0, tile0 + tiles).
  const int per_split = kSplit ? (all_tiles + splits - 1) / splits : all_tiles;
  const int tile0 = kSplit ? min(all_tiles, split * per_split) : 0;
  const int tiles = kSplit ? min(all_tiles, tile0 + per_split) - tile0 : all_tiles;

  KvStager<T, NDT, kVector> stager;
  if (!kSplit || tiles > 0) {  // a split may own no tile of a causal block
    stager.load(kh, vh, tile0 * L::kKeys, S, D);
    stager.store(lds);
  }
  __syncthreads();

  for (int tile = 0; tile < tiles; ++tile) {
    const unsigned char* stage = lds + (tile & 1) * L::kStageBytes;
    const int key0 = (tile0 + tile) * L::kKeys;
    if (tile + 1 < tiles) stager.load(kh, vh, key0 + L::kKeys, S, D);

    const bool wave_active = !causal || key0 <= wave_row0 + kRowsPerWave - 1;
    if (wave_active) {
      // ---- S^T = K Q^T for NKB 32-key tiles --------------------------------
      floatx16 s[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
        const unsigned char* krow = stage + (32 * kb + l32) * L::kKPitch;
#pragma unroll
        for (int c = 0; c < L::kChunkPairs; ++c) {
          const Chunk a =
              *reinterpret_cast<const Chunk*>(krow + (2 * c + half) * 16);
          Pr::mma(s[kb], a, qf[c]);
        }
      }
      // ---- online softmax (log2 domain) --------------------------------------
      const bool needs_mask =
          key0 + L::kKeys > S ||
          (causal && key0 + L::kKeys - 1 > wave_row0);
      float tile_max = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float x = s[kb][e] * score_scale_log2;
          if (needs_mask) {
            const int key = key0 + 32 * kb + 8 * (e / 4) + 4 * half + (e % 4);
            if (key >= S || (causal && key > my_row)) x = -INFINITY;
          }
          s[kb][e] = x;
          tile_max = fmaxf(tile_max, x);
        }
      }
      tile_max = opl::max_lane_xor32(tile_max);
      const float new_max = fmaxf(row_max, tile_max);
      const float alpha = opl::fast_exp2(row_max - new_max);
      row_max = new_max;
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float p = opl::fast_exp2(s[kb][e] - new_max);
          s[kb][e] = p;
          psum += p;
        }
      }
      row_sum = row_sum * alpha + psum;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
      }
      // ---- O^T += V^T P^T -----------------------------------------------------
      const unsigned char* vtile = stage + L::kKBytes;
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            half8 pb;
#pragma unroll
            for (int e = 0; e < 8; ++e)
              pb[e] = static_cast<_Float16>(s[kb][8 * u + e]);
            const int group_byte = (2 * kb + u) * 32 + 16 * half;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
              const half8 a = *reinterpret_cast<const half8*>(
                  vtile + (32 * dt + l32) * L::kVPitch + group_byte);
              o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o[dt], 0,
                                                              0, 0);
            }
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = 8 * (e / 4) + 4 * half + (e % 4);
          const float* vrow =
              reinterpret_cast<const float*>(vtile + key * L::kVPitch);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                vrow[32 * dt + l32], s[0][e], o[dt], 0, 0, 0);
        }
      }
    }

    if (tile + 1 < tiles) stager.store(lds + ((tile + 1) & 1) * L::kStageBytes);
    __syncthreads();
  }

  // ---- normalise and store: lane holds O^T[d][row] for d = 32dt + 8(e/4) +
  // 4*half + e%4, i.e. four runs of 4 consecutive dims per tile ------------
  const float total = opl::sum_lane_xor32(row_sum);
  float inv = 1.0f / total;
  float* out_base = O;
  if constexpr (kSplit) {
    // Partial: unnormalised O, then (max, sum) of the row. A split that saw
    // no visible key of a row leaves max -FLT_MAX, sum 0 and O 0, which
    // the combine weighs by 0.
    inv = 1.0f;
    out_base = part_o + static_cast<std::size_t>(split) * BH * S * D;
    if (my_row < S && half == 0) {
      float* ml = part_ml + (static_cast<std::size_t>(split) * BH * S +
                             static_cast<std::size_t>(bh) * S + my_row) * 2;
      ml[0] = row_max;
      ml[1] = total;
    }
  }
  if (my_row < S) {
    float* orow = out_base + head + static_cast<std::size_t>(my_row) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * dt + 8 * g + 4 * half;
        if constexpr (kVector) {
          if (d0 < D)
            *reinterpret_cast<float4*>(orow + d0) =
                make_float4(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv,
                            o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (d0 + r < D) orow[d0 + r] = o[dt][4 * g + r] * inv;
        }
      }
    }
  }
}

// out[row][d] = sum_s 2^(m_s - m) O_s[row][d] / sum_s 2^(m_s - m) l_s, with
// m = max_s m_s, over the splits in order (deterministic). One thread per
// row and 4 consecutive dims (d0 < D); kVec: D % 4 == 0 and a 16-byte
// aligned output, so the 4 dims move as one float4 (the partials sit in
// the 256-byte aligned workspace).
template <bool kVec>
__global__ __launch_bounds__(256) void attention_combine_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml,
    float* __restrict__ out, long long rows, int D, int splits) {
  const int quads = (D + 3) / 4;
  const long long i = blockIdx.x * 256LL + threadIdx.x;
  if (i >= rows * quads) return;
  const long long row = i / quads;
  const int d0 = static_cast<int>(i % quads) * 4;
  float m = -FLT_MAX;
  for (int sp = 0; sp < splits; ++sp) m = fmaxf(m, part_ml[(sp * rows + row) * 2]);
  float l = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int sp = 0; sp < splits; ++sp) {
    const float w = opl::fast_exp2(part_ml[(sp * rows + row) * 2] - m);
    l += w * part_ml[(sp * rows + row) * 2 + 1];
    const float* o = part_o + (sp * rows + row) * D + d0;
    if constexpr (kVec) {
      const float4v v = *reinterpret_cast<const float4v*>(o);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += w * v[r];
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (d0 + r < D) acc[r] += w * o[r];
    }
  }
  const float inv = 1.0f / l;
  if constexpr (kVec) {
    const float4v v = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
    *reinterpret_cast<float4v*>(out + row * D + d0) = v;
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (d0 + r < D) out[row * D + d0 + r] = acc[r] * inv;
  }
}

// Register-staged kernel (one workgroup per CU): small grids deal each
// query block's keys to `splits` workgroups, as many as keep blocks *
// splits within kSplitBudget workgroups (one per CU), at most 4; causal
// grids, whose heaviest blocks set the time, may use twice that budget.
// Measured on MI355X, fp32 D 128 (us; 1 / 2 / 4 splits): B1 H12 S1024
// 169.6 / 104.0 / 111.9, causal 171.3 / 100.7 / 66.4; B1 H8 S2048 333.0 /
// 194.7 / 205.4; B1 H24 S1024 causal 175.1 / 110.7 / 119.3; B2 H12 S1024
// 175.8 / 198.0 / 174.7.
constexpr long long kSplitBudget = 256;
constexpr int kMaxSplits = 4;

// Key splits of a register-staged call and the scratch bytes of their
// partials: `splits` as above, fewer when the partials would not fit
// `capacity` (one split needs none).
struct SplitPlan {
  int splits = 1;
  std::size_t bytes = 0;
};

template <typename T, int NDT>
SplitPlan split_plan(int bh, int s, int d, int causal, std::size_t capacity) {
  const int q_blocks = (s + kBlockRows - 1) / kBlockRows;
  const long long blocks = static_cast<long long>(q_blocks) * bh;
  // Key tiles per query block bound the useful split count.
  const int max_tiles = (s + AttnLayout<T, NDT>::kKeys - 1) / AttnLayout<T, NDT>::kKeys;
  const long long budget = causal ? 2 * kSplitBudget : kSplitBudget;
  int splits = static_cast<int>(budget / blocks < kMaxSplits ? budget / blocks : kMaxSplits);
  if (splits > max_tiles) splits = max_tiles;
  if (splits < 1) splits = 1;
  const std::size_t per_split =
      static_cast<std::size_t>(bh) * s * (d + 2) * sizeof(float);
  if (splits > 1 && static_cast<std::size_t>(splits) > capacity / per_split)
    splits = static_cast<int>(capacity / per_split);
  SplitPlan p;
  p.splits = splits < 2 ? 1 : splits;
  p.bytes = p.splits > 1 ? per_split * p.splits : 0;
  return p;
}

// Runs the register-staged kernel; `scratch` holds plan.bytes.
template <typename T, int NDT>
hipError_t launch_attention(const T* q, const T* k, const T* v, float* out, int bh,
                            int s, int d, int causal, bool vector_ok, const SplitPlan& plan,
                            void* scratch, hipStream_t stream) {
  const int q_blocks = (s + kBlockRows - 1) / kBlockRows;
  const long long blocks = static_cast<long long>(q_blocks) * bh;
  const float scale = 1.4426950408889634f / sqrtf(static_cast<float>(d));
  const int splits = plan.splits;
  float* part_o = nullptr;
  float* part_ml = nullptr;
  if (splits > 1) {
    const std::size_t rows = static_cast<std::size_t>(bh) * s;
    part_o = static_cast<float*>(scratch);
    part_ml = part_o + static_cast<std::size_t>(splits) * rows * d;
  }
  const dim3 grid(static_cast<unsigned>(blocks * splits)), block(kThreads);
  if (splits > 1) {
    if (vector_ok)
      attention_mfma_kernel<T, NDT, true, true><<<grid, block, 0, stream>>>(
          q, k, v, out, bh, s, d, causal, scale, splits, part_o, part_ml);
    else
      attention_mfma_kernel<T, NDT, false, true><<<grid, block, 0, stream>>>(
          q, k, v, out, bh, s, d, causal, scale, splits, part_o, part_ml);
  } else {
    if (vector_ok)
      attention_mfma_kernel<T, NDT, true, false><<<grid, block, 0, stream>>>(
          q, k, v, out, bh, s, d, causal, scale, 1, nullptr, nullptr);
    else
      attention_mfma_kernel<T, NDT, false, false><<<grid, block, 0, stream>>>(
          q, k, v, out, bh, s, d, causal, scale, 1, nullptr, nullptr);
  }
  if (splits > 1) {
    const long long rows = static_cast<long long>(bh) * s;
    const long long threads = rows * ((d + 3) / 4);
    const dim3 cgrid(static_cast<unsigned>((threads + 255) / 256));
    if (d % 4 == 0 && opl::aligned16(out))
      attention_combine_kernel<true><<<cgrid, dim3(256), 0, stream>>>(
          part_o, part_ml, out, rows, d, splits);
    else
      attention_combine_kernel<false><<<cgrid, dim3(256), 0, stream>>>(
          part_o, part_ml, out, rows, d, splits);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// attention_f16_dma_kernel — fp16 fast path (head_dim 64 or 128, any S,
// 16-byte aligned tensors). Same maths as attention_mfma_kernel; its running
// max moves lazily (below) and its row sums add the fp16-rounded p that P.V
// uses, so results agree up to rounding. What changes:
//   * v_mfma_f32_16x16x32_f16 instead of 32x32x16: the same flops per LDS
//     byte, but the GPU holds a higher clock under the power limit with it.
//     A wavefront's 32 query rows are two 16-row blocks (qc); S^T = K Q^T
//     comes in 16 x 16 blocks, so lane l holds query 16 qc + l % 16 and keys
//     4 (l / 16) + e of each 16-key block; a row's keys span four lanes;
//   * K / V tiles are copied global -> LDS by buffer loads with the lds
//     modifier (buffer_load_dwordx4 ... lds: no VGPR staging, no ds_write,
//     no register transpose of V); the tile's position is a scalar offset;
//   * V stays [key][d] in LDS; its V^T MFMA operand is read with
//     ds_read_b64_tr_b16 (within each 16-lane group, lane 4r + j addresses 4
//     dims of key row r, lane i receives dim i of rows r = 0..3), which also
//     realises the key order of the P^T accumulator registers;
//   * XOR-swizzled 16-byte chunks keep every LDS read conflict-free: K rows
//     use chunk ^ (row & 15) (D = 128) or ^ ((row >> 1) & 7) (D = 64), V rows
//     chunk ^ (4 (row & 3) ^ 2 ((row >> 2) & 1)) / ^ 2 ((row >> 1) & 3); the
//     swizzle terms are lane constants, so per-tile offsets fold into
//     instruction immediates;
//   * row sums on the matrix cores (ones x P^T), one rescale decision per
//     64-key tile;
//   * ~250 VGPRs and 64 KiB of LDS, so two 4-wavefront workgroups share a CU
//     (the LDS is the limit): one wavefront's softmax VALU work overlaps
//     the other's MFMAs.
// Measured on MI355X, B4 H32 S8192 D128 causal: 2.07 ms (1060 TFLOP/s
// effective; 2.23 ms with 32x32x16 MFMAs and VALU row sums), vs 474 TFLOP/s
// for PyTorch's SDPA on the same box.
// ---------------------------------------------------------------------------

namespace dma {

typedef __fp16 fp16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
#define OPL_LDS __attribute__((address_space(3)))

constexpr int kXcds = 8;
// Workgroup slots of an XCD the causal work order is balanced over (32 CUs,
// two workgroups each). Simulated greedy dispatch over 64 slots, B4 H32
// S2048 causal (16 blocks per head of 4..64 32-key tiles, 256 per XCD):
// head-major order finishes at 172 tile-times per slot against the 136
// average; groups of 4 heads, heaviest first, at 136.
constexpr int kCausalGroupSlots = 64;
// Grids of fewer query blocks than this split each block's keys in two:
// up to 256 (a CU each) any grid gains, as the unsplit block runs one
// wavefront per SIMD; causal grids gain up to 384 blocks, because the split
// halves the key walk of their heaviest blocks. Measured on MI355X (us,
// unsplit vs split): B1 H12 S1024 22.1 vs 20.5 (causal 22.1 vs 20.7); B1
// H12 S2048 39.9 vs 36.2; B1 H8 S4096 (256 blocks) 86.1 vs 72.3; B1 H16
// S2048 42.1 vs 38.5, causal 39.8 vs 35.6; B1 H12 S4096 (384) 111.7 vs
// 124.4, causal 102.8 vs 77.2; B1 H32 S2048 (512) 77.5 vs 85.0, causal
// 61.0 vs 63.6; B4 H32 S8192 causal 2238 vs 2408.
constexpr long long kSplitKeysBelow = 257;
constexpr long long kSplitKeysBelowCausal = 512;
// Grids of at most this many 128-row query blocks run 64-row blocks, so
// that twice as many CUs share the work. Measured on MI355X (us, 128- vs
// 64-row blocks, two key groups in both): B1 H12 S1024 20.6 vs 17.6
// (causal 20.6 vs 17.5); B1 H8 S2048 34.0 vs 30.0; B1 H4 S512 causal 13.2
// vs 10.7; past 128 blocks the 64-row grid needs more than one workgroup
// per CU: B1 H12 S2048 (192) 35.5 vs 55.3.
// At D = 128 these grids split keys four ways (four groups of two
// wavefronts on 32-key tiles, two wavefronts per SIMD instead of one), so
// one wavefront's exponentials overlap another's MFMAs. Measured on MI355X
// (us, two groups on 64-key tiles vs four on 32-key tiles, inputs cycling
// past the Infinity Cache): B1 H12 S1024 20.5 vs 19.4 (causal 20.6 vs
// 17.9); B1 H8 S2048 35.4 vs 31.7 (causal 34.6 vs 27.3); B1 H4 S512 11.0
// vs 11.4 (causal 11.2 vs 11.5).
constexpr long long kHalfRowsUpTo = 128;
// D = 64 workgroups hold 64 KiB of LDS (two per CU), so 64-row blocks pay
// off on larger grids. Measured (us, 128- vs 64-row blocks): B1 H32 S1024
// (256 blocks) 17.4 vs 15.2; B1 H12 S4096 (384) 75.9 vs 72.5, causal 48.5
// vs 47.5; B1 H16 S4096 (512) 84.7 vs 90.5, causal (128-row keys unsplit)
// 73.1 vs 52.9. These limits cover every grid that would split keys on
// 128-row blocks, so D = 64 never runs that instance.
constexpr long long kHalfRowsUpToD64 = 384;
constexpr long long kHalfRowsUpToD64Causal = 512;
static_assert(kHalfRowsUpToD64 >= kSplitKeysBelow - 1 &&
                  kHalfRowsUpToD64Causal >= kSplitKeysBelowCausal - 1,
              "every D = 64 grid that splits keys runs 64-row blocks");
// Sequences of at most this many tokens on grids past kHalfRowsUpTo blocks
// run 64-row blocks of two wavefronts on 32-key tiles (16 or 32 KiB of LDS
// instead of 64): a 128-row block held 128 rows for S of them, and its LDS
// let two workgroups share a CU, so launches of many short heads ran in
// latency-bound rounds. Measured on MI355X, fp16 (us, before -> after;
// SDPA): B128 H32 S16 D128 45.3 -> 21.5 (15.2); B16 H32 S1 7.9 -> 6.0
// (12.7); S = 128 was no faster (B32 H32 S128 30.9 vs 32.6).
constexpr int kShortSequence = 64;
// Headroom (log2 units) the running row max may lag the true max by.
constexpr float kLazyLog2 = 8.0f;

// K/V tile layout in LDS for element type T (rows keep their global
// layout, D elements each).
template <typename T, int D, int kTileKeys>
struct Layout {
  static constexpr int kSize = static_cast<int>(sizeof(T));
  static constexpr int kElems = 16 / kSize;  // elements per 16-byte chunk
  static constexpr int kRowBytes = D * kSize;
  static constexpr int kChunks = kRowBytes / 16;
  static constexpr int kTile = kTileKeys * kRowBytes;  // one K or V tile
  static constexpr int kStage = 2 * kTile;
  // QK^T fragment steps over d: one 16-byte chunk per lane group covers 32
  // fp16 dims (one MFMA 16x16x32) or 16 fp32 dims (four MFMA 16x16x4).
  static constexpr int kSubK = 4 * kElems;
  static constexpr int kSteps = D / kSubK;
  static constexpr int kDBlocks = D / 16;  // 16-dim blocks of O^T
  // K rows: 16 consecutive rows read one logical chunk (one 16-lane group)
  // and land on 16 different physical chunks.
  __device__ static int swizzle_k(int row) {
    return kChunks >= 16 ? (row & 15) : ((row >> 1) & 7);
  }
  // V rows, fp16: a ds_read_b64_tr_b16 group reads 8 bytes from each of 4
  // rows (4 lanes per row); the 4 rows, and the next group's 4, land on
  // different banks. fp32: each 16-lane group of a ds_read_b32 reads 64
  // bytes of one row, the four groups rows 4 apart, which land on four
  // different 64-byte bank ranges.
  __device__ static int swizzle_v(int row) {
    if constexpr (kSize == 2)
      return D == 128 ? ((4 * (row & 3)) ^ (2 * ((row >> 2) & 1))) : 2 * ((row >> 1) & 3);
    else
      return 4 * ((row >> 2) & 3);
  }
};

// Scores of one 32-key half for a wavefront's 32 query rows: [kb][qc] is
// the 16 x 16 block of keys 16 kb.. and queries 16 qc.. (S^T layout: lane l
// holds query l % 16, keys 4 (l / 16) + e).
struct HalfScores {
  floatx4 v[2][2];
};

// kGroups > 1 (small grids): kGroups groups of kW wavefronts share the
// workgroup's query rows and split its key tiles into contiguous ranges,
// each group with its own K/V stages; at the end the groups merge their
// (O, max, sum) through LDS in group order, every wavefront taking a share
// of the rows.
// kW = wavefronts per group, 32 query rows each: 4 (128-row blocks), or 2
// (64-row blocks) for the smallest grids, whose 128-row blocks would leave
// CUs idle.
// kTileKeys = keys per K/V tile: 64 (two 32-key halves per tile), or 32,
// which halves the stages so that four groups fit the LDS of two.
// A D = 128 workgroup with two groups and 64-key tiles, or four groups and
// 32-key tiles, holds 128 KiB of LDS (a CU): with kW = 2 that is one or two
// wavefronts per SIMD. The other instances run two wavefronts per SIMD.
// Two K/V stages per group: the copies of tile t + 1 are issued while tile t
// is processed. Rings of three and four 32-key stages per group (copies
// issued two or three tiles ahead, partial vmcnt waits, bare barriers)
// measured no faster on small grids (B1 H12 S1024: 20.9 us for both
// against 20.5 us for two 64-key stages), so the tile loop is not waiting
// on its copies; four groups, two wavefronts per SIMD, are what helps.
// fp32 rows are twice as long: its instances use 32-key tiles (64 KiB of
// K/V stages per group at D = 128), and at most two groups.
// Wavefronts per SIMD an instance must fit: one when four wavefronts hold
// more than half a CU's LDS, else two.
template <typename T, int D, int kGroups, int kW, int kTileKeys>
constexpr int kMinWavesPerSimd =
    2 * kGroups * Layout<T, D, kTileKeys>::kStage > 80 * 1024 && kGroups * kW == 4 ? 1 : 2;

template <typename T, int D, int kGroups, int kW, int kTileKeys>
__global__ __launch_bounds__(kW * opl::kWaveSize * kGroups)
__attribute__((amdgpu_waves_per_eu(kMinWavesPerSimd<T, D, kGroups, kW, kTileKeys>, 2)))
void attention_dma_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                          const T* __restrict__ V, float* __restrict__ O, int BH, int S,
                          int dm, int causal, float score_scale_log2) {
  using L = Layout<T, D, kTileKeys>;
  constexpr bool kHalf = L::kSize == 2;
  using Frag = typename std::conditional<kHalf, half8, floatx4>::type;
  static_assert(kGroups == 1 || kGroups == 2 || kGroups == 4, "1, 2 or 4 key groups");
  static_assert(kW == 2 || kW == 4, "2 or 4 wavefronts per group");
  static_assert(kTileKeys == 32 || kTileKeys == 64, "32- or 64-key tiles");
  constexpr int kRows = kW * kRowsPerWave;  // query rows per workgroup
  // 16-byte copies per lane and tile: the group's lanes share each tile
  constexpr int kCopies = L::kTile / 16 / (kW * opl::kWaveSize);
  constexpr int kArray = kGroups * L::kStage;  // bytes of each stage array
  __shared__ __attribute__((aligned(1024))) unsigned char stage0[kArray];
  __shared__ __attribute__((aligned(1024))) unsigned char stage1[kArray];

  // Work item w = (head, query block) in head-major order, heaviest query
  // block first within a head. Workgroups are dealt to the 8 XCDs
  // round-robin; XCD x takes the contiguous range of work items
  // [x * per_xcd, (x + 1) * per_xcd), so the workgroups resident on one XCD
  // at a time belong to one or two heads and share that head's K/V tiles
  // in the XCD's L2 instead of streaming them from HBM per query block.
  // The last block of a head may run past S: its rows from S on load row
  // S - 1 of Q and are not stored; keys from S on read zeros (the buffer
  // range ends at the head) and are masked.
  const int q_blocks = (S + kRows - 1) / kRows;
  const int total = q_blocks * BH;
  const int per_xcd = (total + kXcds - 1) / kXcds;
  const int w = static_cast<int>(blockIdx.x % kXcds) * per_xcd +
                static_cast<int>(blockIdx.x / kXcds);
  if (w >= total) return;  // padding of the grid to a multiple of 8
  int bh = w / q_blocks;
  int qb = q_blocks - 1 - w % q_blocks;
  // Causal grids with few query blocks per head: a head's blocks (heaviest
  // first) are too few for an XCD's workgroup slots to even out, and the
  // heavy first blocks of the last heads start late. Groups of g heads,
  // g * q_blocks about the slots of an XCD, are taken heaviest first
  // across the group instead (block q_blocks - 1 of each head, then the
  // next): the order a longest-first schedule of the group would use, with
  // as many heads in flight per XCD as before. g = 1 (64 or more blocks
  // per head) keeps the head-major order.
  if (causal) {
    const int g = max(1, kCausalGroupSlots / q_blocks);
    if (g > 1) {
      const int first = w / (g * q_blocks) * g;  // first head of w's group
      const int heads = min(g, BH - first);
      const int r = w - first * q_blocks;        // < heads * q_blocks
      bh = first + r % heads;
      qb = q_blocks - 1 - r / heads;
    }
  }
  const int q0 = qb * kRows;
  const int lane = threadIdx.x % opl::kWaveSize;
  // (Kept as a vector value: declaring it wave-uniform turns the causal
  // tests into scalar branches and measured ~8% slower.)
  const int wave = (threadIdx.x / opl::kWaveSize) % kW;
  const int group = kGroups == 1 ? 0 : __builtin_amdgcn_readfirstlane(
                                           threadIdx.x / opl::kWaveSize / kW);
  unsigned char* const st0 = stage0 + group * L::kStage;
  unsigned char* const st1 = stage1 + group * L::kStage;
  // v_mfma_f32_16x16x32_f16 lane roles: lane l supplies row / column
  // l % 16 of its operands and their 8-element k chunk l / 16; its
  // accumulator holds column l % 16, rows 4 (l / 16) + e, e = 0..3.
  const int col = lane % 16;
  const int quad = lane / 16;
  const int wave_row0 = q0 + wave * kRowsPerWave;
  // dm: the tensors' head dim (memory rows of dm elements); D >= dm is the
  // LDS layout's. Dims from dm on are zeros in Q and in the K/V tiles (their
  // products add nothing) and are not stored.
  const std::size_t head = static_cast<std::size_t>(bh) * S * dm;
  const T* qh = Q + head;
  const T* kh = K + head;
  const T* vh = V + head;

  // Q^T operand of query block qc: query wave_row0 + 16 qc + col, the
  // 16-byte chunk quad of step c (dims kSubK c + kElems quad ..).
  Frag qf[2][L::kSteps];
#pragma unroll
  for (int qc = 0; qc < 2; ++qc)
#pragma unroll
    for (int c = 0; c < L::kSteps; ++c) {
      const int dim = L::kSubK * c + L::kElems * quad;
      qf[qc][c] = *reinterpret_cast<const Frag*>(
          qh + static_cast<std::size_t>(min(wave_row0 + 16 * qc + col, S - 1)) * dm +
          (dim < dm ? dim : 0));
      if (dim >= dm) qf[qc][c] = Frag{};
    }

  // DMA: byte offset of the chunk this lane copies, per copy. Chunks of
  // dims from dm on take an offset past every range (the launcher keeps
  // padded heads under 2^31 bytes), so they read zeros.
  constexpr int kNoData = static_cast<int>(0x80000000u);
  int k_src[kCopies], v_src[kCopies];
#pragma unroll
  for (int j = 0; j < kCopies; ++j) {
    const int slot = (wave * kCopies + j) * 64 + lane;
    const int row = slot / L::kChunks;
    const int phys = slot % L::kChunks;
    const int kd = L::kElems * (phys ^ L::swizzle_k(row));
    const int vd = L::kElems * (phys ^ L::swizzle_v(row));
    k_src[j] = kd < dm ? (row * dm + kd) * L::kSize : kNoData;
    v_src[j] = vd < dm ? (row * dm + vd) * L::kSize : kNoData;
  }
  // Buffer resources over the rest of this head's K and V from the tile's
  // first key (the launcher guarantees S * dm * sizeof(T) < 2^32): the per-lane byte
  // offsets stay in 32-bit VGPRs and the base is scalar, so a tile's copies
  // cost no vector address arithmetic. The hardware range-checks only the
  // per-lane offset against the resource's size (the scalar offset is
  // exempt), so the tile's position goes into the base, not the scalar
  // offset: keys from S on then fall outside the range and read zeros,
  // never the next head or memory past the tensor.
  const unsigned head_bytes = static_cast<unsigned>(S) * dm * L::kSize;
  // The copies' LDS destinations (M0) are wave-uniform: derived from a
  // scalar copy of the wave index, they stay in scalar registers instead of
  // costing a v_readfirstlane per copy and tile.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](unsigned char* st, int key0) {
    // key0 < S for every issued tile, so 0 < rest <= head_bytes < 2^32
    const unsigned tile_bytes = static_cast<unsigned>(key0) * dm * L::kSize;
    const unsigned rest = head_bytes - tile_bytes;
    const std::size_t tile_elems = static_cast<std::size_t>(key0) * dm;
#pragma unroll
    for (int j = 0; j < kCopies; ++j)
      opl::buffer_copy16_lds(kh + tile_elems, rest, st + (wave_s * kCopies + j) * 1024,
                             k_src[j]);
#pragma unroll
    for (int j = 0; j < kCopies; ++j)
      opl::buffer_copy16_lds(vh + tile_elems, rest,
                             st + L::kTile + (wave_s * kCopies + j) * 1024, v_src[j]);
  };
  // K operand: key row col of each 16-key block, chunk 4 c + quad. Rows 16
  // apart share the swizzle, so the block and half offsets are immediates.
  int k_off[L::kSteps];
#pragma unroll
  for (int c = 0; c < L::kSteps; ++c)
    k_off[c] = col * L::kRowBytes + (((4 * c + quad) ^ L::swizzle_k(col)) * 16);
  // V^T operand of dim block db. fp16: lane l addresses 4 dims (16 db + 4
  // (col % 4) ..) of key row 4 quad + col / 4 and receives dim 16 db + col
  // of key rows 4 quad + 0..3 (k slots 8 quad + 0..3); the read 16 rows on
  // gives slots 8 quad + 4..7. fp32: lane l reads dim 16 db + col of key
  // row 4 quad + e for MFMA e (rows 4 quad + e share row 4 quad's
  // swizzle). Either way that is the key order of the P^T registers below.
  int v_base[L::kDBlocks];
#pragma unroll
  for (int db = 0; db < L::kDBlocks; ++db) {
    if constexpr (kHalf) {
      const int row = 4 * quad + col / 4;
      const int d = 16 * db + 4 * (col % 4);
      v_base[db] = L::kTile + row * L::kRowBytes +
                   (((d >> 3) ^ L::swizzle_v(row)) * 16) + (d & 7) * 2;
    } else {
      const int row = 4 * quad;
      const int d = 16 * db + col;
      v_base[db] = L::kTile + row * L::kRowBytes +
                   (((d >> 2) ^ L::swizzle_v(row)) * 16) + (d & 3) * 4;
    }
  }

  // O^T of query block qc, dim block db: lane l holds query 16 qc + col,
  // dims 16 db + 4 quad + e.
  floatx4 o[2][L::kDBlocks];
#pragma unroll
  for (int qc = 0; qc < 2; ++qc)
#pragma unroll
    for (int db = 0; db < L::kDBlocks; ++db)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[qc][db][e] = 0.0f;
  // Online-softmax state of the lane's two query rows.
  float row_max[2] = {-FLT_MAX, -FLT_MAX};
  // Raw score above which the running max must move; -inf until the first
  // visible score.
  float move_above[2] = {-INFINITY, -INFINITY};
  // Row sums on the matrix cores: an all-ones A operand times P^T gives
  // every accumulator row the column sums of P^T, i.e. each lane the full
  // sum of its query row's p (as rounded to fp16 for P.V) in all four
  // elements. That replaces 32 VALU adds per tile and a wavefront with 4
  // MFMAs (the vector ALUs, not the matrix cores, are the busier pipe).
  // fp32 keeps them on the vector ALUs instead (the matrix cores are its
  // busier pipe): each lane sums its 8 of the row's p per 32 keys, and the
  // four lanes of a row are combined once, after the loop.
  floatx4 sums[2];
#pragma unroll
  for (int qc = 0; qc < 2; ++qc)
#pragma unroll
    for (int e = 0; e < 4; ++e) sums[qc][e] = 0.0f;
  float lane_sum[2] = {0.0f, 0.0f};
  half8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = static_cast<_Float16>(1.0f);
  const float inv_scale = 1.0f / score_scale_log2;
  const int visible_end = causal ? min(S, q0 + kRows) : S;
  const int tiles = (visible_end + kTileKeys - 1) / kTileKeys;
  // This group's tiles [t_begin, t_begin + t_count), a contiguous range of
  // at most `iters`; every group runs `iters` iterations so that all meet
  // at every barrier.
  const int iters = (tiles + kGroups - 1) / kGroups;
  const int t_begin = group * iters;
  const int t_count = kGroups == 1 ? tiles : max(0, min(iters, tiles - t_begin));

  auto tile = [&](const unsigned char* cur, unsigned char* nxt, int i) {
    const int key0 = (t_begin + i) * kTileKeys;
    if (i + 1 < t_count) issue(nxt, key0 + kTileKeys);
    __builtin_amdgcn_sched_barrier(0);
    if ((kGroups == 1 || i < t_count) &&
        (!causal || key0 <= wave_row0 + kRowsPerWave - 1)) {
      // A 64-key tile is processed as two 32-key halves. Lazy rescaling
      // (below) lets half 1 be exponentiated against the running max before
      // its own max is checked (it is recomputed in the rare case the max
      // must move), so one basic block holds the scores of half 1, the P.V
      // product of half 0 (matrix cores) and the exponentials of both
      // halves (vector ALUs), and the scheduler can interleave them. A
      // 32-key tile is one such half.
      auto scores = [&](int j) {
        HalfScores s;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qc = 0; qc < 2; ++qc)
#pragma unroll
            for (int e = 0; e < 4; ++e) s.v[kb][qc][e] = 0.0f;
        if constexpr (kHalf) {
          half8 a[2][L::kSteps];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int c = 0; c < L::kSteps; ++c)
              a[kb][c] = *reinterpret_cast<const half8*>(
                  cur + k_off[c] + (32 * j + 16 * kb) * L::kRowBytes);
          // All K reads of the half are issued before the MFMAs: with one
          // workgroup per CU (small grids) nothing else hides their latency.
          __builtin_amdgcn_sched_barrier(0);
          // Four independent accumulators, so no MFMA waits on the previous.
#pragma unroll
          for (int c = 0; c < L::kSteps; ++c)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
              for (int qc = 0; qc < 2; ++qc)
                s.v[kb][qc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    a[kb][c], qf[qc][c], s.v[kb][qc], 0, 0, 0);
        } else {
          // fp32: 16 MFMAs per 16-dim step (4 dims x 2 key blocks x 2
          // query blocks) hide the next step's two K reads.
#pragma unroll
          for (int c = 0; c < L::kSteps; ++c) {
            floatx4 a[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
              a[kb] = *reinterpret_cast<const floatx4*>(
                  cur + k_off[c] + (32 * j + 16 * kb) * L::kRowBytes);
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
              for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int qc = 0; qc < 2; ++qc)
                  s.v[kb][qc] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                      a[kb][e], qf[qc][c][e], s.v[kb][qc], 0, 0, 0);
          }
        }
        return s;
      };
      auto mask = [&](HalfScores& s, int j) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qc = 0; qc < 2; ++qc)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int key = key0 + 32 * j + 16 * kb + 4 * quad + e;
              if ((causal && key > wave_row0 + 16 * qc + col) || key >= S)
                s.v[kb][qc][e] = -INFINITY;
            }
      };
      // Max of this lane's 8 raw scores of query block qc in a half. The
      // row's other 24 sit in lanes l ^ 16, l ^ 32, l ^ 48; they are
      // combined only when the max has to move (move_max).
      auto lane_max = [&](const HalfScores& s, int qc) {
        float m = s.v[0][qc][0];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = kb == 0 ? 1 : 0; e < 4; ++e)
            m = __builtin_elementwise_maximum(m, s.v[kb][qc][e]);
        return m;
      };
      // Lazy rescaling: the running max m (log2 units) only moves when a
      // row's max exceeds it by more than kLazyLog2, so p = 2^(x - m) stays
      // <= 2^kLazyLog2 (well inside fp16's range) and the O rescale is
      // skipped on almost every half-tile. Softmax is shift-invariant: the
      // result is the same up to rounding. The test compares raw scores
      // with move_above = (m + kLazyLog2) / scale, updated when m moves.
      auto needs_move = [&](float raw0, float raw1) {
        return __builtin_amdgcn_ballot_w64(raw0 > move_above[0] ||
                                           raw1 > move_above[1]) != 0;
      };
      // Wave-uniform branch: every lane runs it, and the four lanes of a
      // row combine their maxima, so they move to the same max.
      auto move_max = [&](float raw0, float raw1) {
        const float lane_raw[2] = {raw0, raw1};
#pragma unroll
        for (int qc = 0; qc < 2; ++qc) {
          const float raw = opl::max_lane_xor32(
              opl::combine_xor16_f32<opl::MaxOp>(lane_raw[qc]));
          const float new_max = fmaxf(row_max[qc], raw * score_scale_log2);
          const float alpha = opl::fast_exp2(row_max[qc] - new_max);
          row_max[qc] = new_max;
          move_above[qc] = (new_max + kLazyLog2) * inv_scale;
          if constexpr (kHalf) {
#pragma unroll
            for (int e = 0; e < 4; ++e) sums[qc][e] *= alpha;
          } else {
            lane_sum[qc] *= alpha;
          }
#pragma unroll
          for (int db = 0; db < L::kDBlocks; ++db)
#pragma unroll
            for (int e = 0; e < 4; ++e) o[qc][db][e] *= alpha;
        }
      };
      // P of query block qc as the B operand of P.V. fp16: k slots 8 quad
      // + e are keys 4 quad + e of block 0, slots 8 quad + 4 + e those of
      // block 1. fp32: [qc][kb][e] is key 16 kb + 4 quad + e, the operand of
      // MFMA e over key block kb; the lane's sum of them is kept.
      using PHalf = typename std::conditional<kHalf, half8[2], floatx4[2][2]>::type;
      auto exponentiate = [&](const HalfScores& s, PHalf& pb) {
#pragma unroll
        for (int qc = 0; qc < 2; ++qc)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float p = opl::fast_exp2(
                  fmaf(s.v[kb][qc][e], score_scale_log2, -row_max[qc]));
              if constexpr (kHalf) {
                pb[qc][4 * kb + e] = static_cast<_Float16>(p);
              } else {
                pb[qc][kb][e] = p;
                lane_sum[qc] += p;
              }
            }
      };
      auto accumulate = [&](int j, const PHalf& pb) {
        const int rows = 32 * j * L::kRowBytes;
        if constexpr (!kHalf) {
          // Each O^T accumulator is reused 16 MFMAs after its last update.
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float va[L::kDBlocks];
#pragma unroll
              for (int db = 0; db < L::kDBlocks; ++db)
                va[db] = *reinterpret_cast<const float*>(
                    cur + v_base[db] + rows + (16 * kb + e) * L::kRowBytes);
#pragma unroll
              for (int db = 0; db < L::kDBlocks; ++db)
#pragma unroll
                for (int qc = 0; qc < 2; ++qc)
                  o[qc][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[db], pb[qc][kb][e],
                                                                   o[qc][db], 0, 0, 0);
            }
        } else {
#pragma unroll
          for (int db = 0; db < L::kDBlocks; ++db) {
            const fp16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (OPL_LDS fp16x4*)(cur + v_base[db] + rows));
            const fp16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                (OPL_LDS fp16x4*)(cur + v_base[db] + rows + 16 * L::kRowBytes));
            half8 a;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              a[e] = lo[e];
              a[4 + e] = hi[e];
            }
#pragma unroll
            for (int qc = 0; qc < 2; ++qc)
              o[qc][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[qc], o[qc][db], 0, 0, 0);
          }
#pragma unroll
          for (int qc = 0; qc < 2; ++qc)
            sums[qc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb[qc], sums[qc], 0, 0, 0);
        }
      };
      // One rescale decision per tile, taken on both halves' maxima before
      // either P.V: the O rescale then happens in O's own registers (a
      // second decision after the first P.V made the compiler copy all 64
      // accumulators on every tile that did not rescale). Measured on
      // MI355X, B4 H32 S8192 causal: 2234 -> 2120 us; with the row sums on
      // the matrix cores, 2075 us.
      auto body = [&](auto masked_tag) {
        constexpr bool kMasked = decltype(masked_tag)::value;
        PHalf p0, p1;
        // The QK^T MFMAs of both halves issue at raised wave priority: the
        // SIMD's other wavefront, usually in its exponentials then, yields
        // issue slots to them, so the two wavefronts' matrix and vector
        // phases overlap more. Measured on MI355X (us, B4 H32 S8192 causal /
        // B4 H32 S2048): 2126 -> 2076 / 264.5 -> 258.9 with the priority,
        // 2127 / 262.5 with the same instruction order and no priority;
        // priority 3 instead of 1: 2091 / 258.8. Results bit-identical.
        __builtin_amdgcn_s_setprio(1);
        HalfScores s0 = scores(0);
        HalfScores s1;
        if constexpr (kTileKeys == 64) s1 = scores(1);
        __builtin_amdgcn_s_setprio(0);
        if constexpr (kMasked) mask(s0, 0);
        float a0 = lane_max(s0, 0);
        float a1 = lane_max(s0, 1);
        if constexpr (kTileKeys == 64) {
          if constexpr (kMasked) mask(s1, 1);
          a0 = __builtin_elementwise_maximum(a0, lane_max(s1, 0));
          a1 = __builtin_elementwise_maximum(a1, lane_max(s1, 1));
        }
        if (needs_move(a0, a1)) move_max(a0, a1);
        exponentiate(s0, p0);
        accumulate(0, p0);
        if constexpr (kTileKeys == 64) {
          exponentiate(s1, p1);
          accumulate(1, p1);
        }
      };
      // Only tiles crossing the diagonal or the end of the keys are masked
      // (a wave-uniform test).
      if ((causal && key0 + kTileKeys - 1 > wave_row0) || key0 + kTileKeys > S)
        body(std::true_type{});
      else
        body(std::false_type{});
    }
    __builtin_amdgcn_s_waitcnt(0);  // this tile's reads and the next DMA
    __syncthreads();
  };

  if (t_count > 0) issue(st0, t_begin * kTileKeys);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int i = 0;
  for (; i + 1 < iters; i += 2) {
    tile(st0, st1, i);
    tile(st1, st0, i + 1);
  }
  if (i < iters) tile(st0, st1, i);
  float row_sum[2];
#pragma unroll
  for (int qc = 0; qc < 2; ++qc) {
    if constexpr (kHalf)
      row_sum[qc] = sums[qc][0];
    else  // the four lanes of the row: l, l ^ 16, l ^ 32, l ^ 48
      row_sum[qc] = opl::sum_lane_xor32(opl::combine_xor16_f32<opl::SumOp>(lane_sum[qc]));
  }

  // After the loop every stage is free (the last iteration ended with a
  // barrier and issued no copy). Merge and staging blocks tile the two
  // stage arrays: block (g, w) holds wavefront w of group g's 32 rows of O,
  // 32 * D floats.
  constexpr int kBlockBytes = 2 * L::kDBlocks * 16 * opl::kWaveSize;
  static_assert(kArray % kBlockBytes == 0 && kW * kBlockBytes <= 2 * kArray,
                "blocks tile the two stage arrays");
  auto block = [&](int index) -> float4* {
    const int byte = index * kBlockBytes;
    return reinterpret_cast<float4*>(byte < kArray ? stage0 + byte : stage1 + (byte - kArray));
  };
  // Key-split groups (kGroups > 1): every wavefront merges and stores a
  // share of the rows. (1) Each writes its rows' (max, sum) to LDS; (2)
  // each computes, for its rows, the common max M, the total sum L =
  // sum_g l_g 2^(m_g - M) (groups in order) and its own weight
  // 2^(m - M) / L; (3) each writes its O times that weight to LDS block
  // (group, wave) in the row-major staging layout used for the store
  // below; (4) each of the kGroups * kW wavefronts sums the kGroups copies
  // of 32 / kGroups rows in group order and stores them as whole rows. A
  // group that saw no visible key has max -FLT_MAX and sum 0: weight 0.
  // Against handing every group's state to group 0 in turn (its two
  // wavefronts merging and storing all 64 rows): B1 H12 S1024 16.4 ->
  // 15.4 us, causal 15.8 -> 14.7 us on MI355X.
  if constexpr (kGroups > 1) {
    constexpr int kSlots = kGroups * kW * opl::kWaveSize;
    float* const xs = reinterpret_cast<float*>(stage0);
    const int slot = (group * kW + wave) * opl::kWaveSize + lane;
#pragma unroll
    for (int qc = 0; qc < 2; ++qc) {
      xs[qc * kSlots + slot] = row_max[qc];
      xs[(2 + qc) * kSlots + slot] = row_sum[qc];
    }
    __syncthreads();
    float coef[2];
#pragma unroll
    for (int qc = 0; qc < 2; ++qc) {
      float mg[kGroups], lg[kGroups];
#pragma unroll
      for (int g = 0; g < kGroups; ++g) {
        const int sl = (g * kW + wave) * opl::kWaveSize + lane;
        mg[g] = xs[qc * kSlots + sl];
        lg[g] = xs[(2 + qc) * kSlots + sl];
      }
      float m = mg[0];
#pragma unroll
      for (int g = 1; g < kGroups; ++g) m = fmaxf(m, mg[g]);
      float l = 0.0f;
#pragma unroll
      for (int g = 0; g < kGroups; ++g) l += lg[g] * opl::fast_exp2(mg[g] - m);
      coef[qc] = opl::fast_exp2(row_max[qc] - m) / l;
    }
    __syncthreads();
    constexpr int kChunks4 = D / 4;
    {
      float4* const stg = block(group * kW + wave);
#pragma unroll
      for (int qc = 0; qc < 2; ++qc)
#pragma unroll
        for (int db = 0; db < L::kDBlocks; ++db) {
          const int r = 16 * qc + col;
          const int c = 4 * db + quad;
          stg[r * kChunks4 + (c ^ (r % kChunks4))] =
              make_float4(o[qc][db][0] * coef[qc], o[qc][db][1] * coef[qc],
                          o[qc][db][2] * coef[qc], o[qc][db][3] * coef[qc]);
        }
    }
    __syncthreads();
    constexpr int kWaveRows = kRowsPerWave / kGroups;
    constexpr int kRowsPerStore = opl::kWaveSize / kChunks4;
    static_assert(kWaveRows % kRowsPerStore == 0, "whole store passes");
    const int v = group * kW + wave;
    const int bw = v / kGroups;
    const int r0 = (v % kGroups) * kWaveRows;
    const int rr = lane / kChunks4;
    const int cc = lane % kChunks4;
    float* const obase = O + head + static_cast<std::size_t>(q0 + kRowsPerWave * bw) * dm;
#pragma unroll
    for (int i = 0; i < kWaveRows / kRowsPerStore; ++i) {
      const int row = r0 + kRowsPerStore * i + rr;
      const int idx = row * kChunks4 + (cc ^ (row % kChunks4));
      float4 x = block(bw)[idx];
#pragma unroll
      for (int g = 1; g < kGroups; ++g) {
        const float4 y = block(g * kW + bw)[idx];
        x.x += y.x;
        x.y += y.y;
        x.z += y.z;
        x.w += y.w;
      }
      const float4v xv = {x.x, x.y, x.z, x.w};
      if (q0 + kRowsPerWave * bw + row < S && 4 * cc < dm)
        __builtin_nontemporal_store(xv, reinterpret_cast<float4v*>(obase + static_cast<std::size_t>(row) * dm) + cc);
    }
    return;
  }

  // One group: O leaves through LDS so that every store instruction writes
  // whole rows: the accumulator gives a lane 4 consecutive dims of one row
  // per float4 (a store straight from it writes 16-byte pieces of 16 rows);
  // re-read from the wave's own block, one float4 instruction covers
  // 64 / (D / 4) whole rows. Float4 c of row r sits at position
  // c ^ (r % (D / 4)): both the writes (16 rows, one float4 position each)
  // and the reads (one row per 32 or 16 lanes) spread over the banks.
  float inv[2];
#pragma unroll
  for (int qc = 0; qc < 2; ++qc)
    inv[qc] = 1.0f / row_sum[qc];
  {
    constexpr int kChunks4 = D / 4;  // float4s per output row
    float4* const stg = block(wave);
#pragma unroll
    for (int qc = 0; qc < 2; ++qc)
#pragma unroll
      for (int db = 0; db < L::kDBlocks; ++db) {
        const int r = 16 * qc + col;
        const int c = 4 * db + quad;
        stg[r * kChunks4 + (c ^ (r % kChunks4))] =
            make_float4(o[qc][db][0] * inv[qc], o[qc][db][1] * inv[qc],
                        o[qc][db][2] * inv[qc], o[qc][db][3] * inv[qc]);
      }
    constexpr int kRowsPerStore = opl::kWaveSize / kChunks4;
    const int rr = lane / kChunks4;
    const int cc = lane % kChunks4;
    float* const obase = O + head + static_cast<std::size_t>(wave_row0) * dm;
#pragma unroll
    for (int i = 0; i < kRowsPerWave / kRowsPerStore; ++i) {
      const int row = kRowsPerStore * i + rr;
      const float4 x = stg[row * kChunks4 + (cc ^ (row % kChunks4))];
      const float4v xv = {x.x, x.y, x.z, x.w};
      if (wave_row0 + row < S && 4 * cc < dm)
        __builtin_nontemporal_store(xv, reinterpret_cast<float4v*>(obase + static_cast<std::size_t>(row) * dm) + cc);
    }
  }
}

#undef OPL_LDS
}  // namespace dma

// True when the fast path applies: aligned tensors whose head dim is 64 or
// 128, or any other whole number of 16-byte chunks up to 128, which runs
// the instances of the next of 64 and 128 with the dims past it zero (its
// K/V chunks take an out-of-range offset of 2^31 bytes, so such heads must
// stay below that).
inline int dma_layout(int head_dim) { return head_dim <= 64 ? 64 : 128; }

inline bool dma_ok(const void* q, const void* k, const void* v, const void* out,
                   int sequence, int head_dim, unsigned element_bytes) {
  // one head of K or V must be addressable with 32-bit buffer offsets
  const unsigned long long head_bytes =
      static_cast<unsigned long long>(sequence) * head_dim * element_bytes;
  const bool native = head_dim == 64 || head_dim == 128;
  const bool padded = !native && head_dim <= 128 &&
                      head_dim % static_cast<int>(16 / element_bytes) == 0 &&
                      head_bytes < (1ull << 31);
  return (native ? head_bytes < (1ull << 32) : padded) &&
         opl::aligned16(q) && opl::aligned16(k) && opl::aligned16(v) &&
         opl::aligned16(out);
}

template <typename T>
int attention_entry(const T* q, const T* k, const T* v, float* out, int batch,
                    int heads, int sequence, int head_dim, int causal,
                    const opl::ScratchSource& src, std::size_t* query,
                    void* stream_handle) {
  if (!opl::attention_args_ok(q, k, v, out, batch, heads, sequence, head_dim))
    return hipErrorInvalidValue;
  const int bh = batch * heads;
  const long long blocks =
      static_cast<long long>((sequence + kBlockRows - 1) / kBlockRows) * bh;
  if (blocks > 0x7fffffffLL - 8) return hipErrorInvalidValue;
  constexpr int E = 16 / sizeof(T);
  const bool vector_ok = head_dim % E == 0 && opl::aligned16(q) &&
                         opl::aligned16(k) && opl::aligned16(v) &&
                         opl::aligned16(out);
  hipStream_t stream = static_cast<hipStream_t>(stream_handle);
  const int c = causal ? 1 : 0;
  if (dma_ok(q, k, v, out, sequence, head_dim, sizeof(T))) {
    if (query != nullptr) {  // the fast path needs no scratch
      *query = 0;
      return hipSuccess;
    }
    const float scale = 1.4426950408889634f / sqrtf(static_cast<float>(head_dim));
    // Grids too small to fill the CUs split each query block's keys
    // between groups of wavefronts in the workgroup; the smallest also
    // halve the query block (and, fp16 at D = 128, split its keys four ways).
    const int layout = dma_layout(head_dim);
    const long long half_up_to =
        layout == 128 ? dma::kHalfRowsUpTo
                        : (causal ? dma::kHalfRowsUpToD64Causal : dma::kHalfRowsUpToD64);
    const bool half_rows = blocks <= half_up_to;
    const bool split = half_rows ||
        blocks < (causal ? dma::kSplitKeysBelowCausal : dma::kSplitKeysBelow);
    const long long wgs = half_rows ? 2 * blocks : blocks;
    // a multiple of 8 workgroups, one contiguous range of work per XCD
    const long long padded = (wgs + dma::kXcds - 1) / dma::kXcds * dma::kXcds;
    const dim3 grid(static_cast<unsigned>(padded));
    if constexpr (sizeof(T) == 2) {
      if (sequence <= dma::kShortSequence && !half_rows) {
        const long long tb = (sequence + 63) / 64 * static_cast<long long>(bh);
        const long long tw = (tb + dma::kXcds - 1) / dma::kXcds * dma::kXcds;
        const dim3 tgrid(static_cast<unsigned>(tw));
        if (layout == 128)
          dma::attention_dma_kernel<T, 128, 1, 2, 32><<<tgrid, dim3(kThreads / 2), 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        else
          dma::attention_dma_kernel<T, 64, 1, 2, 32><<<tgrid, dim3(kThreads / 2), 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        return hipGetLastError();
      }
      if (layout == 128) {
        // 64-row blocks x 4 groups / 128-row blocks x 2 groups: 8 wavefronts
        const dim3 block(split ? 2 * kThreads : kThreads);
        if (half_rows)
          dma::attention_dma_kernel<T, 128, 4, 2, 32><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        else if (split)
          dma::attention_dma_kernel<T, 128, 2, 4, 64><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        else
          dma::attention_dma_kernel<T, 128, 1, 4, 64><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
      } else {
        // (split implies half_rows at D = 64; 4 wavefronts either way)
        const dim3 block(kThreads);
        if (half_rows)
          dma::attention_dma_kernel<T, 64, 2, 2, 64><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        else
          dma::attention_dma_kernel<T, 64, 1, 4, 64><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
      }
    } else {
      // fp32: 32-key tiles, at most two groups (a group's K/V stages hold
      // 64 KiB at D = 128): 64-row blocks with two groups of 2 wavefronts,
      // 128-row blocks with two groups of 4, or one group of 4.
      if (layout == 128) {
        const dim3 block(split && !half_rows ? 2 * kThreads : kThreads);
        if (half_rows)
          dma::attention_dma_kernel<T, 128, 2, 2, 32><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        else if (split)
          dma::attention_dma_kernel<T, 128, 2, 4, 32><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        else
          dma::attention_dma_kernel<T, 128, 1, 4, 32><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
      } else {
        const dim3 block(kThreads);
        if (half_rows)
          dma::attention_dma_kernel<T, 64, 2, 2, 32><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
        else
          dma::attention_dma_kernel<T, 64, 1, 4, 32><<<grid, block, 0, stream>>>(
              q, k, v, out, bh, sequence, head_dim, c, scale);
      }
    }
    return hipGetLastError();
  }
  const int ndt = (head_dim + 31) / 32;
  SplitPlan plan;
  switch (ndt) {
    case 1: plan = split_plan<T, 1>(bh, sequence, head_dim, c, src.capacity()); break;
    case 2: plan = split_plan<T, 2>(bh, sequence, head_dim, c, src.capacity()); break;
    case 3: plan = split_plan<T, 3>(bh, sequence, head_dim, c, src.capacity()); break;
    default: plan = split_plan<T, 4>(bh, sequence, head_dim, c, src.capacity()); break;
  }
  if (query != nullptr) {
    *query = plan.bytes;
    return hipSuccess;
  }
  if (src.workspace_mode && !opl::workspace_ok(src.data, src.bytes, plan.bytes))
    return hipErrorInvalidValue;
  auto run = [&](void* scratch) -> hipError_t {
    switch (ndt) {
      case 1: return launch_attention<T, 1>(q, k, v, out, bh, sequence, head_dim, c, vector_ok, plan, scratch, stream);
      case 2: return launch_attention<T, 2>(q, k, v, out, bh, sequence, head_dim, c, vector_ok, plan, scratch, stream);
      case 3: return launch_attention<T, 3>(q, k, v, out, bh, sequence, head_dim, c, vector_ok, plan, scratch, stream);
      default: return launch_attention<T, 4>(q, k, v, out, bh, sequence, head_dim, c, vector_ok, plan, scratch, stream);
    }
  };
  if (plan.bytes == 0) return run(nullptr);
  // Held until the combine kernel is enqueued (scratch.hpp).
  opl::ScratchLease lease(stream, src.workspace_mode ? src.data : nullptr, src.bytes);
  if (lease.status() != hipSuccess) return lease.status();
  return run(lease.data());
}

const _Float16* as_f16(const operatorlib_half_t* p) {
  return reinterpret_cast<const _Float16*>(p);
}

}  // namespace

extern "C" int operatorlib_attention_f32(const float* q, const float* k,
                                         const float* v, float* output,
                                         int batch, int heads, int sequence,
                                         int head_dim, int causal,
                                         void* stream_handle) {
  return attention_entry<float>(q, k, v, output, batch, heads, sequence, head_dim, causal,
                                opl::ScratchSource{}, nullptr, stream_handle);
}

extern "C" int operatorlib_attention_f16(const operatorlib_half_t* q,
                                         const operatorlib_half_t* k,
                                         const operatorlib_half_t* v,
                                         float* output, int batch, int heads,
                                         int sequence, int head_dim,
                                         int causal, void* stream_handle) {
  return attention_entry<_Float16>(as_f16(q), as_f16(k), as_f16(v), output, batch, heads,
                                   sequence, head_dim, causal, opl::ScratchSource{}, nullptr,
                                   stream_handle);
}

// Workspace queries: the same plan as the call with these arguments,
// nothing enqueued; invalid arguments report 0.
extern "C" size_t operatorlib_attention_f32_workspace_size(const float* q, const float* k,
                                                           const float* v,
                                                           const float* output, int batch,
                                                           int heads, int sequence,
                                                           int head_dim, int causal) {
  std::size_t bytes = 0;
  if (attention_entry<float>(q, k, v, const_cast<float*>(output), batch, heads, sequence,
                             head_dim, causal, opl::ScratchSource{true, nullptr, 0}, &bytes,
                             nullptr) != hipSuccess)
    return 0;
  return bytes;
}

extern "C" size_t operatorlib_attention_f16_workspace_size(const operatorlib_half_t* q,
                                                           const operatorlib_half_t* k,
                                                           const operatorlib_half_t* v,
                                                           const float* output, int batch,
                                                           int heads, int sequence,
                                                           int head_dim, int causal) {
  std::size_t bytes = 0;
  if (attention_entry<_Float16>(as_f16(q), as_f16(k), as_f16(v), const_cast<float*>(output),
                                batch, heads, sequence, head_dim, causal,
                                opl::ScratchSource{true, nullptr, 0}, &bytes,
                                nullptr) != hipSuccess)
    return 0;
  return bytes;
}

extern "C" int operatorlib_attention_f32_ws(const float* q, const float* k, const float* v,
                                            float* output, int batch, int heads, int sequence,
                                            int head_dim, int causal, void* workspace,
                                            size_t workspace_bytes, void* stream_handle) {
  return attention_entry<float>(q, k, v, output, batch, heads, sequence, head_dim, causal,
                                opl::ScratchSource{true, workspace, workspace_bytes}, nullptr,
                                stream_handle);
}

extern "C" int operatorlib_attention_f16_ws(const operatorlib_half_t* q,
                                            const operatorlib_half_t* k,
                                            const operatorlib_half_t* v, float* output,
                                            int batch, int heads, int sequence, int head_dim,
                                            int causal, void* workspace, size_t workspace_bytes,
                                            void* stream_handle) {
  return attention_entry<_Float16>(as_f16(q), as_f16(k), as_f16(v), output, batch, heads,
                                   sequence, head_dim, causal,
                                   opl::ScratchSource{true, workspace, workspace_bytes}, nullptr,
                                   stream_handle);
}
