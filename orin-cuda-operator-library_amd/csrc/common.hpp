#pragma once
// Device-side building blocks shared by the operatorlib kernels (gfx950,
// 64-lane wavefronts).
//
// Cross-lane reductions use the CDNA data-parallel primitives instead of
// generic shuffles: DPP quad permutes and row mirrors combine lanes inside a
// 16-lane row, v_permlane16_swap (gfx950, register to register) combines the
// two rows of each 32-lane half, and two v_readlane_b32 combine the halves
// into a wave-uniform scalar. Every step is a full butterfly, so all lanes see identical bits and
// the result is independent of scheduling (bitwise deterministic).
//
// The reductions require all 64 lanes to be active: callers pad inactive
// elements with the operation's identity instead of branching around the
// call.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace opl {

constexpr int kWaveSize = 64;

// DPP control words (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <-> 7-i within 8 lanes
constexpr int kDppRowMirror = 0x140;     // lane i <-> 15-i within 16 lanes

template <int Ctrl>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, Ctrl, 0xF, 0xF, false);
}

template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, dpp_i32<Ctrl>(__builtin_bit_cast(int, v)));
}

template <int Ctrl>
__device__ __forceinline__ double dpp_f64(double v) {
  const std::uint64_t bits = __builtin_bit_cast(std::uint64_t, v);
  const int lo = dpp_i32<Ctrl>(static_cast<int>(bits & 0xffffffffu));
  const int hi = dpp_i32<Ctrl>(static_cast<int>(bits >> 32));
  const std::uint64_t out = (static_cast<std::uint64_t>(
                                 static_cast<std::uint32_t>(hi))
                             << 32) |
                            static_cast<std::uint32_t>(lo);
  return __builtin_bit_cast(double, out);
}

// The value of lane l ^ 16 as the pair (own row's value, partner row's
// value) in both lanes: v_permlane16_swap with both operands v returns
// rows (0, 0, 2, 2) and (1, 1, 3, 3) of v. Op::apply on the pair gives
// the lane ^ 16 combination with the lower row's value first in every lane.
template <class Op>
__device__ __forceinline__ float combine_xor16_f32(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return Op::apply(__builtin_bit_cast(float, static_cast<unsigned>(r[0])),
                   __builtin_bit_cast(float, static_cast<unsigned>(r[1])));
}

__device__ __forceinline__ double sum_xor16_f64(double v) {
  const std::uint64_t bits = __builtin_bit_cast(std::uint64_t, v);
  const unsigned lo = static_cast<unsigned>(bits & 0xffffffffu);
  const unsigned hi = static_cast<unsigned>(bits >> 32);
  const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  const double a = __builtin_bit_cast(
      double, (static_cast<std::uint64_t>(static_cast<unsigned>(rh[0])) << 32) |
                  static_cast<unsigned>(rl[0]));
  const double b = __builtin_bit_cast(
      double, (static_cast<std::uint64_t>(static_cast<unsigned>(rh[1])) << 32) |
                  static_cast<unsigned>(rl[1]));
  return a + b;
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const std::uint64_t bits = __builtin_bit_cast(std::uint64_t, v);
  const std::uint32_t lo = static_cast<std::uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(bits & 0xffffffffu), lane));
  const std::uint32_t hi = static_cast<std::uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(bits >> 32), lane));
  return __builtin_bit_cast(double,
                            (static_cast<std::uint64_t>(hi) << 32) | lo);
}

struct SumOp {
  template <typename T>
  __device__ __forceinline__ static T apply(T a, T b) {
    return a + b;
  }
};

struct MaxOp {
  __device__ __forceinline__ static float apply(float a, float b) {
    return fmaxf(a, b);
  }
};

// Wave-wide all-reduce; every lane receives the same (uniform) value.
template <class Op>
__device__ __forceinline__ float wave_reduce(float v) {
  v = Op::apply(v, dpp_f32<kDppQuadXor1>(v));
  v = Op::apply(v, dpp_f32<kDppQuadXor2>(v));
  v = Op::apply(v, dpp_f32<kDppRowHalfMirror>(v));
  v = Op::apply(v, dpp_f32<kDppRowMirror>(v));
  v = combine_xor16_f32<Op>(v);
  return Op::apply(readlane_f32(v, 0), readlane_f32(v, 32));
}

__device__ __forceinline__ double wave_reduce_sum_f64(double v) {
  v += dpp_f64<kDppQuadXor1>(v);
  v += dpp_f64<kDppQuadXor2>(v);
  v += dpp_f64<kDppRowHalfMirror>(v);
  v += dpp_f64<kDppRowMirror>(v);
  v = sum_xor16_f64(v);
  return readlane_f64(v, 0) + readlane_f64(v, 32);
}

// Block-wide all-reduce over `Waves` wavefronts through a small LDS array
// (`slots` must hold `Waves` floats and must not be reused by the caller
// until after the next __syncthreads()). Partial results are combined in
// wave order, so the result is deterministic.
template <class Op, int Waves>
__device__ __forceinline__ float block_reduce(float v, float* slots) {
  v = wave_reduce<Op>(v);
  if constexpr (Waves == 1) {
    return v;
  } else {
    const int wave = threadIdx.x / kWaveSize;
    if ((threadIdx.x % kWaveSize) == 0) slots[wave] = v;
    __syncthreads();
    float r = slots[0];
#pragma unroll
    for (int w = 1; w < Waves; ++w) r = Op::apply(r, slots[w]);
    return r;
  }
}

// 2^x on the hardware transcendental unit (v_exp_f32). Callers fold log2(e)
// into their arguments so that exp(x) costs one FMA plus one v_exp_f32.
__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

constexpr float kLog2e = 1.4426950408889634f;

// Alignment test for the 16-byte vector paths.
__host__ __device__ inline bool aligned16(const void* p) {
  return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0;
}

// Word 3 of a raw (untyped, unswizzled) buffer resource on gfx9-family
// parts: 32-bit data format, no index stride; only the byte range matters.
constexpr int kBufferFlags = 0x00020000;

// 16 bytes per lane from base + voffset into LDS at dst + 16 * lane (dst
// wave-uniform), through a buffer resource over [base, base + bytes): the
// base lives in scalar registers, so a copy needs no 64-bit vector address
// arithmetic, and a lane whose offset reaches past `bytes` reads zeros and
// touches no memory. The hardware range-checks only the per-lane offset,
// not the instruction's scalar offset, so this helper passes no scalar
// offset: callers move a tile's position into `base` and shrink `bytes` to
// match. Kept out of kernel bodies so the host compilation pass never meets
// the device-only resource type.
__device__ __forceinline__ void buffer_copy16_lds(const void* base, unsigned bytes,
                                                  unsigned char* dst, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                        bytes, kBufferFlags),
      (__attribute__((address_space(3))) void*)dst, 16, voffset, 0, 0, 0);
}

// max / sum of v over lanes l and l ^ 32 (the two halves of a wavefront),
// the same value in both lanes. v_permlane32_swap exchanges the halves
// register to register, where __shfl_xor(v, 32) is an LDS round trip
// (ds_bpermute). Sums add the lower half's value first in every lane. The
// max is IEEE maximum (NaN-propagating, v_maximum_f32), which needs none
// of the canonicalising moves fmaxf adds.
__device__ __forceinline__ float max_lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace opl
