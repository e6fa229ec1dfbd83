#pragma once
// operatorlib C++ API — signature-compatible drop-in for the reference's
// include/operatorlib/operators.h:13-44 (same names, parameter order and
// defaults), with hipError_t / hipStream_t / __half in place of the CUDA
// types.
//
// All pointers refer to device memory owned by the caller. Launchers enqueue
// work on `stream` and never synchronize the device. They return
// hipErrorInvalidValue for bad arguments (checked before any HIP call) or the
// launch error. Each function is an inline forwarder to the C ABI declared in
// operatorlib/operatorlib_c.h, which is what liboperatorlib.so exports.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstddef>

#include "operatorlib/operatorlib_c.h"

namespace operatorlib {

// Reference: include/operatorlib/operators.h:13
inline hipError_t reduce_sum_f32(const float* input, float* output,
                                 std::size_t n, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_reduce_sum_f32(
      input, output, n, static_cast<void*>(stream)));
}

// Reference: include/operatorlib/operators.h:16
inline hipError_t softmax_f32(const float* input, float* output, int rows,
                              int cols, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_softmax_f32(
      input, output, rows, cols, static_cast<void*>(stream)));
}

// Reference: include/operatorlib/operators.h:19
inline hipError_t transpose_f32(const float* input, float* output, int rows,
                                int cols, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_transpose_f32(
      input, output, rows, cols, static_cast<void*>(stream)));
}

// Reference: include/operatorlib/operators.h:22
inline hipError_t rmsnorm_f32(const float* input, const float* weight,
                              float* output, int tokens, int hidden,
                              float epsilon, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_rmsnorm_f32(
      input, weight, output, tokens, hidden, epsilon,
      static_cast<void*>(stream)));
}

// FP16 rows, FP32 max / exp / sum, FP16 output. Not in the reference API
// (its deferred FP16 extension, docs/pytorch_extension.md:143-146).
inline hipError_t softmax_f16(const __half* input, __half* output, int rows,
                              int cols, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_softmax_f16(
      reinterpret_cast<const operatorlib_half_t*>(input),
      reinterpret_cast<operatorlib_half_t*>(output), rows, cols,
      static_cast<void*>(stream)));
}

// FP16 input / weight / output, FP32 sum of squares and scaling. Not in the
// reference API (its deferred FP16 extension).
inline hipError_t rmsnorm_f16(const __half* input, const __half* weight,
                              __half* output, int tokens, int hidden,
                              float epsilon, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_rmsnorm_f16(
      reinterpret_cast<const operatorlib_half_t*>(input),
      reinterpret_cast<const operatorlib_half_t*>(weight),
      reinterpret_cast<operatorlib_half_t*>(output), tokens, hidden, epsilon,
      static_cast<void*>(stream)));
}

// Row-major C[M,N] = A[M,K] * B[K,N].
// Reference: include/operatorlib/operators.h:27
inline hipError_t gemm_f32(const float* a, const float* b, float* c, int m,
                           int n, int k, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(
      operatorlib_gemm_f32(a, b, c, m, n, k, static_cast<void*>(stream)));
}

// FP16 inputs, FP32 MFMA accumulation and FP32 output.
// Reference: include/operatorlib/operators.h:31
inline hipError_t gemm_f16(const __half* a, const __half* b, float* c, int m,
                           int n, int k, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_gemm_f16(
      reinterpret_cast<const operatorlib_half_t*>(a),
      reinterpret_cast<const operatorlib_half_t*>(b), c, m, n, k,
      static_cast<void*>(stream)));
}

// Q/K/V and output use contiguous [B,H,S,D] row-major storage.
// Reference: include/operatorlib/operators.h:35
inline hipError_t attention_f32(const float* q, const float* k, const float* v,
                                float* output, int batch, int heads,
                                int sequence, int head_dim, bool causal,
                                hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_attention_f32(
      q, k, v, output, batch, heads, sequence, head_dim, causal ? 1 : 0,
      static_cast<void*>(stream)));
}

// FP16 Q/K/V, FP32 online-softmax state and FP32 output.
// Reference: include/operatorlib/operators.h:41
inline hipError_t attention_f16(const __half* q, const __half* k,
                                const __half* v, float* output, int batch,
                                int heads, int sequence, int head_dim,
                                bool causal, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(operatorlib_attention_f16(
      reinterpret_cast<const operatorlib_half_t*>(q),
      reinterpret_cast<const operatorlib_half_t*>(k),
      reinterpret_cast<const operatorlib_half_t*>(v), output, batch, heads,
      sequence, head_dim, causal ? 1 : 0, static_cast<void*>(stream)));
}

}  // namespace operatorlib
