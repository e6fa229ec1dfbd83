// reduce_sum_f32: output[0] = sum of n fp32 values.
//
// Reference behaviour: operatorlib::reduce_sum_f32 (src/reduce.cu:54-69)
// zeroes the output in-stream and combines per-block fp32 partials with
// float atomics, so its summation order (and its last bits) change from run
// to run.
//
// MI355X design (one launch, deterministic, HBM-bound):
//   * each thread streams 16-byte loads, kUnroll of them in flight, over a
//     contiguous chunk of 256 * kUnroll float4 per workgroup iteration;
//   * each float4 is summed in fp32 and accumulated into an fp64 register,
//     so rounding error stays far below the fp32 result ulp even for
//     ill-conditioned (zero-mean) inputs;
//   * wave64 DPP/swizzle fp64 reduction, then 4 wave partials via LDS;
//   * the last workgroup to arrive (arrival counter in library scratch)
//     adds all workgroup partials in index order and writes the fp32 result
//     and re-arms the counter. No memset launch, no float atomics.
// Algorithmic traffic: 4 * n bytes read, 4 bytes written.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "scratch.hpp"
#include "validate.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / opl::kWaveSize;
constexpr int kUnroll = 4;

__device__ __forceinline__ double sum4(const float4& v) {
  return static_cast<double>((v.x + v.y) + (v.z + v.w));
}

// Block-wide fp64 sum in a fixed order; result valid in thread 0.
__device__ __forceinline__ double block_sum_f64(double v, double* slots) {
  v = opl::wave_reduce_sum_f64(v);
  const int wave = threadIdx.x / opl::kWaveSize;
  if ((threadIdx.x % opl::kWaveSize) == 0) slots[wave] = v;
  __syncthreads();
  double total = slots[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) total += slots[w];
  return total;
}

__global__ __launch_bounds__(kThreads) void reduce_sum_kernel(
    const float* __restrict__ input, float* __restrict__ output,
    std::size_t n, std::size_t head, std::size_t nvec, double* partials,
    unsigned* counter) {
  const float4* __restrict__ vin =
      reinterpret_cast<const float4*>(input + head);
  const std::size_t chunk = static_cast<std::size_t>(kThreads) * kUnroll;
  const std::size_t full_chunks = nvec / chunk;
  double acc = 0.0;
  for (std::size_t c = blockIdx.x; c < full_chunks; c += gridDim.x) {
    const float4* p = vin + c * chunk + threadIdx.x;
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) v[u] = p[u * kThreads];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc += sum4(v[u]);
  }
  // Leftover whole vectors (fewer than one chunk).
  for (std::size_t i = full_chunks * chunk +
                       static_cast<std::size_t>(blockIdx.x) * kThreads +
                       threadIdx.x;
       i < nvec; i += static_cast<std::size_t>(gridDim.x) * kThreads)
    acc += sum4(vin[i]);
  // Scalar head (before the first 16-byte boundary) and tail (< 4 values).
  if (blockIdx.x == 0) {
    if (threadIdx.x < head) acc += input[threadIdx.x];
    const std::size_t tail = head + nvec * 4;
    if (tail + threadIdx.x < n) acc += input[tail + threadIdx.x];
  }

  __shared__ double slots[kWaves];
  __shared__ int is_last;
  const double block_total = block_sum_f64(acc, slots);
  if (threadIdx.x == 0) {
    if (gridDim.x == 1) {
      output[0] = static_cast<float>(block_total);
      is_last = 0;
    } else {
      __hip_atomic_store(&partials[blockIdx.x], block_total, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      const unsigned arrived = __hip_atomic_fetch_add(
          counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      is_last = arrived == gridDim.x - 1 ? 1 : 0;
    }
  }
  __syncthreads();
  if (!is_last) return;

  // Last workgroup: every other workgroup's partial is visible once the
  // acquire above is extended to the whole workgroup.
  __threadfence();
  double t = 0.0;
  for (unsigned i = threadIdx.x; i < gridDim.x; i += kThreads)
    t += __hip_atomic_load(&partials[i], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();  // `slots` is reused below
  const double total = block_sum_f64(t, slots);
  if (threadIdx.x == 0) {
    output[0] = static_cast<float>(total);
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

extern "C" int operatorlib_reduce_sum_f32(const float* input, float* output,
                                          size_t n, void* stream_handle) {
  if (!opl::reduce_args_ok(input, output, n)) return hipErrorInvalidValue;
  hipStream_t stream = static_cast<hipStream_t>(stream_handle);
  const std::uintptr_t address = reinterpret_cast<std::uintptr_t>(input);
  std::size_t head = ((16u - (address & 15u)) & 15u) / sizeof(float);
  head = std::min(head, n);
  const std::size_t nvec = (n - head) / 4;
  const std::size_t chunk = static_cast<std::size_t>(kThreads) * kUnroll;
  const std::size_t wanted = std::max<std::size_t>(
      1, (nvec + chunk - 1) / chunk);
  const int blocks = static_cast<int>(
      std::min<std::size_t>(wanted, opl::kReduceMaxBlocks));
  opl::ReduceScratch scratch{nullptr, nullptr};
  if (blocks > 1) {
    const hipError_t status = opl::reduce_scratch_for_stream(stream, &scratch);
    if (status != hipSuccess) return status;
  }
  reduce_sum_kernel<<<blocks, kThreads, 0, stream>>>(
      input, output, n, head, nvec, scratch.partials, scratch.counter);
  return hipGetLastError();
}
