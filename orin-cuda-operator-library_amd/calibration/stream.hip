// HBM streaming calibration kernels (measurement only; not part of the
// operatorlib ABI). bench.py times them beside the operators so that each
// bandwidth figure can be read against what a plain stream achieves on the
// same box, at the same sizes and under the same cold-cache rotation, and
// the PMC traffic runs use the copy as the known-size reference for
// FETCH_SIZE / WRITE_SIZE.
//
//   opl_calib_copy_f32: out[i] = in[i], 16-byte non-temporal loads and
//     stores; 8 bytes of traffic per element;
//   opl_calib_read_f32: reads in[] the same way and writes one float per
//     workgroup (0 unless the sum happens to hit a sentinel, so the loads
//     stay); 4 bytes of traffic per element.
// Shapes: the fastest of a sweep on one MI355X over 256 / 512 / 1024
// threads, 1-8 float4 per thread per step, and one chunk per workgroup or
// a persistent grid of 256-2048 workgroups, at 32, 64 and 128 MiB with
// inputs cycling through 1 GiB: 256 threads, one float4 per thread per
// step, a persistent grid of 1024 (copy) or 2048 (read) workgroups. Copy
// 32 / 64 / 128 MiB each way: 12.18 / 22.36 / 42.41 us (5.51 / 6.00 / 6.33
// TB/s); read 64 MiB: 10.66 us (6.30 TB/s). The slowest shapes took up to
// 1.8x longer.
// n must be a multiple of 4 and both buffers 16-byte aligned (checked).

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

constexpr int kThreads = 256;
constexpr unsigned kCopyGrid = 1024;
constexpr unsigned kReadGrid = 2048;

typedef float float4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void copy_kernel(const float4v* __restrict__ in,
                                                        float4v* __restrict__ out,
                                                        std::size_t nvec) {
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * kThreads;
  for (std::size_t i = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
       i < nvec; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(in + i), out + i);
}

__global__ __launch_bounds__(kThreads) void read_kernel(const float4v* __restrict__ in,
                                                        float* __restrict__ out,
                                                        std::size_t nvec) {
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * kThreads;
  float acc = 0.0f;
  for (std::size_t i = blockIdx.x * static_cast<std::size_t>(kThreads) + threadIdx.x;
       i < nvec; i += stride) {
    const float4v v = __builtin_nontemporal_load(in + i);
    acc += (v[0] + v[1]) + (v[2] + v[3]);
  }
  // A data-dependent store the compiler cannot remove; the sentinel is
  // never hit by the bench's inputs, so the kernel writes one float per
  // workgroup: zero.
  out[blockIdx.x] = acc == 3.0e38f ? acc : 0.0f;
}

bool args_ok(const void* in, const void* out, std::size_t n) {
  return in != nullptr && out != nullptr && n != 0 && n % 4 == 0 &&
         (reinterpret_cast<std::uintptr_t>(in) & 15u) == 0 &&
         (reinterpret_cast<std::uintptr_t>(out) & 15u) == 0;
}

unsigned grid_for(std::size_t nvec, unsigned cap) {
  const std::size_t wanted = (nvec + kThreads - 1) / kThreads;
  return static_cast<unsigned>(wanted < cap ? wanted : cap);
}

}  // namespace

extern "C" int opl_calib_copy_f32(const float* in, float* out, size_t n, void* stream) {
  if (!args_ok(in, out, n)) return hipErrorInvalidValue;
  const std::size_t nvec = n / 4;
  copy_kernel<<<grid_for(nvec, kCopyGrid), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const float4v*>(in), reinterpret_cast<float4v*>(out), nvec);
  return hipGetLastError();
}

// `out` must hold one float per workgroup: opl_calib_read_blocks(n) floats.
extern "C" size_t opl_calib_read_blocks(size_t n) { return grid_for(n / 4, kReadGrid); }

extern "C" int opl_calib_read_f32(const float* in, float* out, size_t n, void* stream) {
  if (!args_ok(in, out, n)) return hipErrorInvalidValue;
  const std::size_t nvec = n / 4;
  read_kernel<<<grid_for(nvec, kReadGrid), kThreads, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const float4v*>(in), out, nvec);
  return hipGetLastError();
}
