// reduce_sum_f32: output[0] = sum of n fp32 values.
//
// Reference behaviour: operatorlib::reduce_sum_f32 (src/reduce.cu:54-69)
// zeroes the output in-stream and combines per-block fp32 partials with
// float atomics, so its summation order (and its last bits) change from run
// to run.
//
// MI355X design (deterministic, HBM-bound):
//   * pass 1: 512-thread workgroups stream 16-byte loads, kUnroll in flight
//     per thread; each float4 is summed in fp32 and accumulated in an fp64
//     register, so rounding error stays far below the fp32 result ulp even
//     for ill-conditioned (zero-mean) inputs; a wave64 DPP/permlane fp64
//     reduction and an 8-slot LDS combine give one fp64 partial per
//     workgroup, written to scratch: the caller's workspace
//     (operatorlib_reduce_sum_f32_ws) or the GPU's arena (scratch.hpp);
//   * pass 2: one workgroup adds the partials in index order and writes the
//     fp32 result (stream order makes pass 1's partials visible).
// Inputs that fit one workgroup skip pass 2. No memset, no float atomics.
//
// operatorlib_reduce_sum_f32_noalloc runs the same two kernels with the
// partials in a file-scope device array of its own (`scratch`, 2 KiB per
// GPU), with no lease: no cross-stream ordering, no host lock.
//
// Why two launches: combining in the same launch needs each workgroup to
// publish its partial at device scope and count arrivals. With a release
// fence that costs an L2 writeback per workgroup (~300 us for 2048
// workgroups); with device-scope stores and one arrival counter the
// arrivals serialize on the counter's address. Measured on one MI355X,
// n = 2^24, inputs cycling through 1 GiB (us per call, median of 6 runs of
// 50 back-to-back calls): pass 1 alone 11.13; pass 1 + combine launch
// 12.89; one launch with an arrival counter 14.07 (256 workgroups) and
// 16.61 (512).
// Algorithmic traffic: 4 * n bytes read, 4 bytes written.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <map>
#include <mutex>

#include "common.hpp"
#include "operatorlib/operatorlib_c.h"
#include "scratch.hpp"
#include "validate.hpp"

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / opl::kWaveSize;
constexpr int kUnroll = 4;
// Pass-1 grid cap: one workgroup per CU, each walking several chunks.
// Measured on MI355X, n = 2^24, inputs cycling through 1 GiB (us, grid cap
// 256 / 512 / 1024): 12.88 / 13.25 / 13.76 with 4 loads in flight per
// thread; 8 or 16 in flight were no faster (13.35-14.14).
constexpr int kGridBlocks = 256;
constexpr int kCombineThreads = 256;

typedef float float4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ double sum4(const float4& v) {
  return static_cast<double>((v.x + v.y) + (v.z + v.w));
}

// Block-wide fp64 sum in a fixed order; every thread gets the result.
template <int Waves>
__device__ __forceinline__ double block_sum_f64(double v, double* slots) {
  v = opl::wave_reduce_sum_f64(v);
  const int wave = threadIdx.x / opl::kWaveSize;
  if ((threadIdx.x % opl::kWaveSize) == 0) slots[wave] = v;
  __syncthreads();
  double total = slots[0];
#pragma unroll
  for (int w = 1; w < Waves; ++w) total += slots[w];
  return total;
}

__global__ __launch_bounds__(kThreads) void reduce_partials_kernel(
    const float* __restrict__ input, float* __restrict__ output,
    std::size_t n, std::size_t head, std::size_t nvec,
    double* __restrict__ partials) {
  const float4* __restrict__ vin =
      reinterpret_cast<const float4*>(input + head);
  const std::size_t chunk = static_cast<std::size_t>(kThreads) * kUnroll;
  const std::size_t full_chunks = nvec / chunk;
  double acc = 0.0;
  for (std::size_t c = blockIdx.x; c < full_chunks; c += gridDim.x) {
    const float4* p = vin + c * chunk + threadIdx.x;
    float4v v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)  // read once: non-temporal (+5% measured)
      v[u] = __builtin_nontemporal_load(reinterpret_cast<const float4v*>(p + u * kThreads));
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      acc += sum4(make_float4(v[u][0], v[u][1], v[u][2], v[u][3]));
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
  const double total = block_sum_f64<kWaves>(acc, slots);
  if (threadIdx.x == 0) {
    if (gridDim.x == 1)
      output[0] = static_cast<float>(total);
    else
      partials[blockIdx.x] = total;
  }
}

__global__ __launch_bounds__(kCombineThreads) void reduce_combine_kernel(
    const double* __restrict__ partials, int count, float* __restrict__ output) {
  double t = 0.0;
  for (int i = threadIdx.x; i < count; i += kCombineThreads) t += partials[i];
  __shared__ double slots[kCombineThreads / opl::kWaveSize];
  const double total =
      block_sum_f64<kCombineThreads / opl::kWaveSize>(t, slots);
  if (threadIdx.x == 0) output[0] = static_cast<float>(total);
}

// Grid of one call: the scalar head before the first 16-byte boundary, the
// float4 body, and the number of pass-1 workgroups (at most kGridBlocks).
struct Plan {
  std::size_t head;
  std::size_t nvec;
  int blocks;
};

Plan plan_for(const float* input, std::size_t n) {
  const std::uintptr_t address = reinterpret_cast<std::uintptr_t>(input);
  Plan p;
  p.head = std::min<std::size_t>(((16u - (address & 15u)) & 15u) / sizeof(float), n);
  p.nvec = (n - p.head) / 4;
  const std::size_t chunk = static_cast<std::size_t>(kThreads) * kUnroll;
  const std::size_t wanted = std::max<std::size_t>(1, (p.nvec + chunk - 1) / chunk);
  p.blocks = static_cast<int>(std::min<std::size_t>(wanted, kGridBlocks));
  return p;
}

// Pass 1 and, for more than one workgroup, pass 2 over `partials` (at least
// p.blocks doubles; unused for one workgroup).
hipError_t enqueue(const float* input, float* output, std::size_t n, const Plan& p,
                   double* partials, hipStream_t stream) {
  reduce_partials_kernel<<<p.blocks, kThreads, 0, stream>>>(input, output, n, p.head,
                                                            p.nvec, partials);
  if (p.blocks > 1)
    reduce_combine_kernel<<<1, kCombineThreads, 0, stream>>>(partials, p.blocks,
                                                             output);
  return hipGetLastError();
}

// Partials of operatorlib_reduce_sum_f32_noalloc: one array per GPU, held
// from the library's load to process exit. A call's pass 1 writes every
// slot pass 2 reads, so nothing in it has to start at zero.
static __device__ __align__(256) double scratch[kGridBlocks];

// Device address of `scratch` on the current device. The name `scratch` in
// host code is a host-side stand-in, so kernels get this address instead;
// it is looked up once per device, with that device current.
hipError_t scratch_on_current_device(double** out) {
  int device = 0;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  static std::mutex mutex;
  static std::map<int, double*> by_device;
  std::lock_guard<std::mutex> lock(mutex);
  const auto found = by_device.find(device);
  if (found != by_device.end()) {
    *out = found->second;
    return hipSuccess;
  }
  double* ptr = nullptr;
  status = hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch));
  if (status != hipSuccess) return status;
  by_device.emplace(device, ptr);
  *out = ptr;
  return hipSuccess;
}

// Scratch bytes of a plan: one fp64 partial per pass-1 workgroup when there
// is more than one.
std::size_t partial_bytes(const Plan& p) {
  return p.blocks > 1 ? sizeof(double) * static_cast<std::size_t>(p.blocks) : 0;
}

// The partials come from the caller's workspace (src.workspace_mode) or the
// arena; either way a plan needs at most 2 KiB, so every plan fits and the
// result bits do not depend on the scratch source.
int reduce_with(const float* input, float* output, std::size_t n,
                const opl::ScratchSource& src, hipStream_t stream) {
  const Plan p = plan_for(input, n);
  const std::size_t bytes = partial_bytes(p);
  if (src.workspace_mode && !opl::workspace_ok(src.data, src.bytes, bytes))
    return hipErrorInvalidValue;
  if (bytes == 0) return enqueue(input, output, n, p, nullptr, stream);
  // Held until the combine kernel is enqueued (scratch.hpp).
  opl::ScratchLease lease(stream, src.workspace_mode ? src.data : nullptr, src.bytes);
  if (lease.status() != hipSuccess) return lease.status();
  double* partials = static_cast<double*>(lease.data());
  reduce_partials_kernel<<<p.blocks, kThreads, 0, stream>>>(input, output, n, p.head, p.nvec,
                                                            partials);
  const hipError_t status = hipGetLastError();
  if (status != hipSuccess) return status;
  return lease.launch_last(reduce_combine_kernel, dim3(1), dim3(kCombineThreads),
                           static_cast<const double*>(partials), p.blocks, output);
}

}  // namespace

extern "C" int operatorlib_reduce_sum_f32(const float* input, float* output,
                                          size_t n, void* stream_handle) {
  if (!opl::reduce_args_ok(input, output, n)) return hipErrorInvalidValue;
  return reduce_with(input, output, n, opl::ScratchSource{},
                     static_cast<hipStream_t>(stream_handle));
}

extern "C" size_t operatorlib_reduce_sum_f32_workspace_size(const float* input, size_t n) {
  return n == 0 ? 0 : partial_bytes(plan_for(input, n));
}

extern "C" int operatorlib_reduce_sum_f32_ws(const float* input, float* output, size_t n,
                                             void* workspace, size_t workspace_bytes,
                                             void* stream_handle) {
  if (!opl::reduce_args_ok(input, output, n)) return hipErrorInvalidValue;
  return reduce_with(input, output, n, opl::ScratchSource{true, workspace, workspace_bytes},
                     static_cast<hipStream_t>(stream_handle));
}

extern "C" int operatorlib_reduce_sum_f32_noalloc(const float* input, float* output,
                                                  size_t n, void* stream_handle) {
  if (!opl::reduce_args_ok(input, output, n)) return hipErrorInvalidValue;
  hipStream_t stream = static_cast<hipStream_t>(stream_handle);
  const Plan p = plan_for(input, n);
  // The grid never exceeds kGridBlocks workgroups, so every n fits the
  // kGridBlocks partials of `scratch`: there is no size to reject.
  static_assert(sizeof(scratch) == sizeof(double) * kGridBlocks, "one slot per workgroup");
  double* partials = nullptr;
  if (p.blocks > 1) {
    const hipError_t status = scratch_on_current_device(&partials);
    if (status != hipSuccess) return status;
  }
  return enqueue(input, output, n, p, partials, stream);
}
