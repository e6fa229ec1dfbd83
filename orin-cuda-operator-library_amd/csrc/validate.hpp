#pragma once
// Argument predicates of every entry point. Pure C++ with no HIP calls, so the
// library rejects bad arguments before it touches the runtime (and the checks
// run, and are tested, on machines without a GPU).
//
// Each predicate mirrors a launcher prologue of the reference:
//   reduce     src/reduce.cu:56-57      softmax   src/softmax.cu:184-185
//   transpose  src/transpose.cu:40-41   rmsnorm   src/rmsnorm.cu:80-82
//   gemm       src/gemm.cu:443-445, :457-459
//   attention  src/attention.cu:448-451, :489-492
// The attention predicate also rejects batch * heads beyond int32, which the
// reference checks only in its torch binding (operatorlib_binding.cpp:164-166)
// but which its launchers silently overflow.

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <limits>

namespace opl {

inline bool reduce_args_ok(const void* input, const void* output,
                           std::size_t n) {
  return input != nullptr && output != nullptr && n != 0;
}

inline bool matrix_args_ok(const void* input, const void* output, int rows,
                           int cols) {
  return input != nullptr && output != nullptr && rows > 0 && cols > 0;
}

inline bool rmsnorm_args_ok(const void* input, const void* weight,
                            const void* output, int tokens, int hidden,
                            float epsilon) {
  // The reference's own predicate, `epsilon <= 0.0f` rejects
  // (src/rmsnorm.cu:80-81): NaN compares false, so a NaN epsilon is accepted
  // and gives NaN rows, as there. (The torch binding rejects non-finite
  // epsilon before it gets here, as the reference's binding does.)
  return input != nullptr && weight != nullptr && output != nullptr &&
         tokens > 0 && hidden > 0 && !(epsilon <= 0.0f);
}

inline bool gemm_args_ok(const void* a, const void* b, const void* c, int m,
                         int n, int k) {
  return a != nullptr && b != nullptr && c != nullptr && m > 0 && n > 0 &&
         k > 0;
}

constexpr int kMaxHeadDim = 128;

inline bool attention_args_ok(const void* q, const void* k, const void* v,
                              const void* output, int batch, int heads,
                              int sequence, int head_dim) {
  if (q == nullptr || k == nullptr || v == nullptr || output == nullptr)
    return false;
  if (batch <= 0 || heads <= 0 || sequence <= 0 || head_dim <= 0 ||
      head_dim > kMaxHeadDim)
    return false;
  return static_cast<std::int64_t>(batch) * heads <=
         std::numeric_limits<int>::max();
}

}  // namespace opl
