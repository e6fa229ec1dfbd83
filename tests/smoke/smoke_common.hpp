// Shared helpers of the HIP smoke programs (tests/smoke/*.cpp).
//
// The programs are C++ callers of the operatorlib C++ API
// (include/operatorlib/operators.h), as the reference's ctest programs
// tests/core_ops_smoke.cu, tests/gemm_smoke.cu and tests/attention_smoke.cu
// are callers of its API. Inputs come from the oracle's SplitMix64 generator
// and expected values from the fp64 oracle (oracle/oracle.h), which is
// linked as the checker. Each check prints "<name>=PASS" or
// "<name>=FAIL ..."; the program prints "<program>=PASS" and exits 0 only
// if every check passed.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "oracle.h"
#include "operatorlib/operators.h"

#define SMOKE_HIP(call)                                                      \
  do {                                                                       \
    const hipError_t smoke_error_ = (call);                                  \
    if (smoke_error_ != hipSuccess) {                                        \
      std::fprintf(stderr, "%s:%d %s -> %s\n", __FILE__, __LINE__, #call,    \
                   hipGetErrorString(smoke_error_));                         \
      std::exit(EXIT_FAILURE);                                               \
    }                                                                        \
  } while (0)

namespace smoke {

inline int& failures() {
  static int count = 0;
  return count;
}

// Device copy of a host vector, freed when it goes out of scope.
template <typename T>
class DeviceArray {
 public:
  explicit DeviceArray(std::size_t n) : n_(n) {
    SMOKE_HIP(hipMalloc(&ptr_, std::max<std::size_t>(n, 1) * sizeof(T)));
  }
  DeviceArray(const std::vector<T>& host, hipStream_t stream)
      : DeviceArray(host.size()) {
    SMOKE_HIP(hipMemcpyAsync(ptr_, host.data(), n_ * sizeof(T),
                             hipMemcpyHostToDevice, stream));
  }
  ~DeviceArray() { (void)hipFree(ptr_); }
  DeviceArray(const DeviceArray&) = delete;
  DeviceArray& operator=(const DeviceArray&) = delete;

  T* get() const { return ptr_; }
  std::vector<T> download(hipStream_t stream) const {
    std::vector<T> host(n_);
    SMOKE_HIP(hipMemcpyAsync(host.data(), ptr_, n_ * sizeof(T),
                             hipMemcpyDeviceToHost, stream));
    SMOKE_HIP(hipStreamSynchronize(stream));
    return host;
  }

 private:
  T* ptr_ = nullptr;
  std::size_t n_;
};

inline std::vector<float> uniform(std::uint64_t seed, std::size_t n, float lo,
                                  float hi) {
  std::vector<float> v(n);
  oracle_fill_uniform(seed, lo, hi, v.data(), n);
  return v;
}

inline std::vector<float> normal(std::uint64_t seed, std::size_t n, float mean,
                                 float stddev) {
  std::vector<float> v(n);
  oracle_fill_normal(seed, mean, stddev, v.data(), n);
  return v;
}

// fp32 -> fp16 bits (round to nearest even); `values` is overwritten with
// the rounded numbers so the fp64 reference sees exactly what the GPU does.
inline std::vector<__half> to_half(std::vector<float>& values) {
  std::vector<std::uint16_t> bits(values.size());
  oracle_f32_to_f16_array(values.data(), bits.data(), values.size());
  oracle_f16_to_f32_array(bits.data(), values.data(), values.size());
  std::vector<__half> out(values.size());
  std::memcpy(out.data(), bits.data(), bits.size() * sizeof(std::uint16_t));
  return out;
}

inline void report(const char* name, bool ok, double error, double bound) {
  std::printf("%s=%s max_error=%.3e bound=%.3e\n", name, ok ? "PASS" : "FAIL",
              error, bound);
  if (!ok) ++failures();
}

inline int finish(const char* program) {
  std::printf("%s=%s\n", program, failures() == 0 ? "PASS" : "FAIL");
  return failures() == 0 ? EXIT_SUCCESS : EXIT_FAILURE;
}

}  // namespace smoke
