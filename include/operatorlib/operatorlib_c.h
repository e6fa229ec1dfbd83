/*
 * operatorlib C ABI — the stable, language-neutral boundary of the library.
 *
 * Every entry point takes device pointers that the caller owns, plain sizes
 * and an opaque stream handle (a hipStream_t cast to void*, NULL = the null
 * stream of the current device).  Each call validates its arguments before
 * touching the HIP runtime, enqueues its kernels on `stream` and returns at
 * once: it never synchronizes the device or the stream.
 *
 * Return value: a hipError_t value as int.  0 (hipSuccess) on success,
 * 1 (hipErrorInvalidValue) for the argument errors listed per function
 * (checked before any HIP call), otherwise the launch error reported by
 * hipGetLastError().  Faults inside a kernel surface at the caller's next
 * synchronization, as with any asynchronous HIP work.
 *
 * Device memory: the library never allocates. Launch sequences that need
 * scratch beyond the caller's buffers (reduce partials, per-segment
 * partials of softmax and RMSNorm rows split over workgroups, split-K
 * partial sums, padded GEMM operands, split attention partials) take it
 * from one of two places:
 *   - the plain entry points: a static array of 256 MiB per GPU (the
 *     "arena"), held from the library's load to process exit. Calls that
 *     use it on different streams are ordered on the device by an event
 *     chain, so they stay safe across streams and host threads without
 *     blocking the host. A plan that would need more than 256 MiB uses
 *     fewer splits or a kernel that needs none. Under stream capture the
 *     chain is not captured: replays of such a graph must not overlap
 *     another arena user on the same GPU (replay in stream order with the
 *     other calls, or capture the *_ws entry points instead);
 *   - the *_ws entry points: a workspace the caller passes (device memory,
 *     256-byte aligned, at least the bytes the matching *_workspace_size
 *     query returns for the same arguments, else hipErrorInvalidValue);
 *     the caller orders its uses. With enough workspace the plan is the
 *     one an unlimited arena would give.
 *
 * The C++ API in operatorlib/operators.h (the drop-in for the reference's
 * include/operatorlib/operators.h:13-44) is a thin inline layer over the
 * plain entry points; the PyTorch binding calls the *_ws entry points with
 * a workspace from torch's caching allocator.
 */
#ifndef OPERATORLIB_OPERATORLIB_C_H_
#define OPERATORLIB_OPERATORLIB_C_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE-754 binary16 bit pattern (the storage of __half / torch.float16). */
typedef uint16_t operatorlib_half_t;

/* Version of this ABI; bumped on any incompatible change. */
#define OPERATORLIB_ABI_VERSION 3
int operatorlib_abi_version(void);

/* Human-readable text for a status returned by any entry point. */
const char* operatorlib_status_string(int status);

/*
 * output[0] = sum(input[0..n)) as fp32.  Overwrites output (no prior zeroing
 * needed).  Deterministic: the same input gives the same bits on every call.
 * Errors: input/output NULL, n == 0.
 * Replaces operatorlib::reduce_sum_f32, reference src/reduce.cu:54-69.
 */
int operatorlib_reduce_sum_f32(const float* input, float* output, size_t n,
                               void* stream);

/*
 * Workspace form of operatorlib_reduce_sum_f32: the partials in `workspace`
 * (see the top of this file). The result bits are those of
 * operatorlib_reduce_sum_f32.
 * Errors: as operatorlib_reduce_sum_f32; a workspace smaller than
 * operatorlib_reduce_sum_f32_workspace_size(input, n), or NULL or not
 * 256-byte aligned when that is non-zero.
 * No counterpart in the reference (its launcher needs no scratch:
 * src/reduce.cu:54-69): for callers that own all device memory.
 */
size_t operatorlib_reduce_sum_f32_workspace_size(const float* input, size_t n);
int operatorlib_reduce_sum_f32_ws(const float* input, float* output, size_t n,
                                  void* workspace, size_t workspace_bytes,
                                  void* stream);

/*
 * operatorlib_reduce_sum_f32 without any allocation: the same kernels and
 * the same result bits, with the per-workgroup partials in a static device
 * array of its own, 256 doubles (2 KiB per GPU, held until the process
 * ends), instead of the arena, and without the arena's host lock and event
 * calls. No hipMalloc, no hipFree, no allocating library call,
 * on any call, so callers that cannot allocate (code under HIP graph
 * capture that forbids it, tight serving loops, harnesses that forbid
 * allocation) can use it. Any n is accepted: the grid is capped at 256
 * workgroups, one partial each.
 * Every call on a GPU shares that GPU's array: calls whose executions
 * overlap on one GPU (different streams, or different host threads) race
 * and may return wrong sums; serialize them (one stream, one thread).
 * Errors: as operatorlib_reduce_sum_f32.
 * No counterpart in the reference: an entry point for callers that cannot
 * allocate.
 */
int operatorlib_reduce_sum_f32_noalloc(const float* input, float* output,
                                       size_t n, void* stream);

/*
 * Row-wise numerically stable softmax of a row-major [rows, cols] matrix.
 * Errors: NULL pointer, rows <= 0, cols <= 0.
 * Replaces operatorlib::softmax_f32, reference src/softmax.cu:182-202.
 */
int operatorlib_softmax_f32(const float* input, float* output, int rows,
                            int cols, void* stream);

/*
 * output[c * rows + r] = input[r * cols + c] (out-of-place, bit-exact).
 * Errors: NULL pointer, rows <= 0, cols <= 0.
 * Replaces operatorlib::transpose_f32, reference src/transpose.cu:38-47.
 */
int operatorlib_transpose_f32(const float* input, float* output, int rows,
                              int cols, void* stream);

/*
 * output[t, h] = input[t, h] * rsqrt(mean_h(input[t, :]^2) + epsilon)
 *                * weight[h]  for a row-major [tokens, hidden] input.
 * Errors: NULL pointer, tokens <= 0, hidden <= 0, epsilon <= 0 (the
 * reference's `epsilon <= 0.0f` test, src/rmsnorm.cu:80-81: a NaN epsilon
 * passes it and gives NaN rows).
 * Replaces operatorlib::rmsnorm_f32, reference src/rmsnorm.cu:77-95.
 */
int operatorlib_rmsnorm_f32(const float* input, const float* weight,
                            float* output, int tokens, int hidden,
                            float epsilon, void* stream);

/*
 * softmax_f32 for fp16 rows: fp16 input and output, max / exp / sum in
 * fp32, each output rounded to fp16 once (round to nearest even).
 * Errors: as operatorlib_softmax_f32.
 * No entry point in the reference: its deferred "FP16 input, FP32
 * accumulation" extension (docs/pytorch_extension.md:143-146,
 * softmax/reports/v4.md:140-141).
 */
int operatorlib_softmax_f16(const operatorlib_half_t* input,
                            operatorlib_half_t* output, int rows, int cols,
                            void* stream);

/*
 * rmsnorm_f32 for fp16 tensors: fp16 input, weight and output; the sum of
 * squares, rsqrt and scaling in fp32, each output rounded to fp16 once.
 * Errors: as operatorlib_rmsnorm_f32.
 * No entry point in the reference: its deferred FP16 extension
 * (docs/pytorch_extension.md:143-146).
 */
int operatorlib_rmsnorm_f16(const operatorlib_half_t* input,
                            const operatorlib_half_t* weight,
                            operatorlib_half_t* output, int tokens,
                            int hidden, float epsilon, void* stream);

/*
 * Workspace forms of the softmax and RMSNorm entry points (see the top of
 * this file). Rows longer than 32768 columns, and fewer than 64 rows longer
 * than 4096, are cut into segments over workgroups whose partials (8 bytes
 * per row and segment for softmax, 4 for RMSNorm) go to scratch; every
 * other shape needs none (the queries return 0). The result bits are those
 * of the plain forms.
 * Errors: as the plain forms; a workspace smaller than the query's answer,
 * or NULL or not 256-byte aligned when that is non-zero. The queries
 * return 0 for invalid sizes.
 * No counterpart in the reference (src/softmax.cu:182-202 and
 * src/rmsnorm.cu:77-95 need no scratch): for callers that own all device
 * memory.
 */
size_t operatorlib_softmax_f32_workspace_size(int rows, int cols);
int operatorlib_softmax_f32_ws(const float* input, float* output, int rows,
                               int cols, void* workspace,
                               size_t workspace_bytes, void* stream);
size_t operatorlib_softmax_f16_workspace_size(int rows, int cols);
int operatorlib_softmax_f16_ws(const operatorlib_half_t* input,
                               operatorlib_half_t* output, int rows, int cols,
                               void* workspace, size_t workspace_bytes,
                               void* stream);
size_t operatorlib_rmsnorm_f32_workspace_size(int tokens, int hidden);
int operatorlib_rmsnorm_f32_ws(const float* input, const float* weight,
                               float* output, int tokens, int hidden,
                               float epsilon, void* workspace,
                               size_t workspace_bytes, void* stream);
size_t operatorlib_rmsnorm_f16_workspace_size(int tokens, int hidden);
int operatorlib_rmsnorm_f16_ws(const operatorlib_half_t* input,
                               const operatorlib_half_t* weight,
                               operatorlib_half_t* output, int tokens,
                               int hidden, float epsilon, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * Row-major C[m, n] = A[m, k] * B[k, n], fp32 in / fp32 out.
 * Errors: NULL pointer, m/n/k <= 0.
 * Replaces operatorlib::gemm_f32, reference src/gemm.cu:440-453.
 */
int operatorlib_gemm_f32(const float* a, const float* b, float* c, int m,
                         int n, int k, void* stream);

/*
 * Row-major C[m, n] = A[m, k] * B[k, n]; fp16 A/B, fp32 accumulation and
 * fp32 C.
 * Errors: NULL pointer, m/n/k <= 0.
 * Replaces operatorlib::gemm_f16, reference src/gemm.cu:455-479.
 */
int operatorlib_gemm_f16(const operatorlib_half_t* a,
                         const operatorlib_half_t* b, float* c, int m, int n,
                         int k, void* stream);

/*
 * Workspace forms of the GEMMs (see the top of this file): the query gives
 * the scratch bytes of the plan for these operands (split partial sums,
 * and padded copies of large fp16 operands whose rows are not 4-byte
 * aligned; 0 for most shapes).
 * Errors: as the plain forms; a workspace smaller than the query's answer,
 * or NULL or not 256-byte aligned when that is non-zero.
 * No counterpart in the reference (src/gemm.cu:440-479 needs no scratch):
 * for callers that own all device memory.
 */
size_t operatorlib_gemm_f32_workspace_size(const float* a, const float* b,
                                           int m, int n, int k);
int operatorlib_gemm_f32_ws(const float* a, const float* b, float* c, int m,
                            int n, int k, void* workspace,
                            size_t workspace_bytes, void* stream);
size_t operatorlib_gemm_f16_workspace_size(const operatorlib_half_t* a,
                                           const operatorlib_half_t* b,
                                           int m, int n, int k);
int operatorlib_gemm_f16_ws(const operatorlib_half_t* a,
                            const operatorlib_half_t* b, float* c, int m,
                            int n, int k, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * output = softmax(Q K^T / sqrt(head_dim) [+ causal mask]) V for contiguous
 * [batch, heads, sequence, head_dim] fp32 tensors; causal != 0 hides key j
 * from query row i when j > i.
 * Errors: NULL pointer, any size <= 0, head_dim > 128,
 *         batch * heads > INT32_MAX.
 * Replaces operatorlib::attention_f32, reference src/attention.cu:445-484.
 */
int operatorlib_attention_f32(const float* q, const float* k, const float* v,
                              float* output, int batch, int heads,
                              int sequence, int head_dim, int causal,
                              void* stream);

/*
 * As operatorlib_attention_f32 with fp16 Q/K/V, fp32 scores, fp32
 * online-softmax state and fp32 output.
 * Replaces operatorlib::attention_f16, reference src/attention.cu:486-507.
 */
int operatorlib_attention_f16(const operatorlib_half_t* q,
                              const operatorlib_half_t* k,
                              const operatorlib_half_t* v, float* output,
                              int batch, int heads, int sequence,
                              int head_dim, int causal, void* stream);

/*
 * Workspace forms of the attention entry points (see the top of this
 * file): key-split partials of small register-staged grids; the fp16 fast
 * path (head_dim 64 or 128, 16-byte aligned tensors) needs none.
 * Errors: as the plain forms; a workspace smaller than the query's answer,
 * or NULL or not 256-byte aligned when that is non-zero. The queries
 * return 0 for invalid arguments.
 * No counterpart in the reference (src/attention.cu:445-507 needs no
 * scratch): for callers that own all device memory.
 */
size_t operatorlib_attention_f32_workspace_size(const float* q, const float* k,
                                                const float* v,
                                                const float* output, int batch,
                                                int heads, int sequence,
                                                int head_dim, int causal);
int operatorlib_attention_f32_ws(const float* q, const float* k,
                                 const float* v, float* output, int batch,
                                 int heads, int sequence, int head_dim,
                                 int causal, void* workspace,
                                 size_t workspace_bytes, void* stream);
size_t operatorlib_attention_f16_workspace_size(const operatorlib_half_t* q,
                                                const operatorlib_half_t* k,
                                                const operatorlib_half_t* v,
                                                const float* output, int batch,
                                                int heads, int sequence,
                                                int head_dim, int causal);
int operatorlib_attention_f16_ws(const operatorlib_half_t* q,
                                 const operatorlib_half_t* k,
                                 const operatorlib_half_t* v, float* output,
                                 int batch, int heads, int sequence,
                                 int head_dim, int causal, void* workspace,
                                 size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* OPERATORLIB_OPERATORLIB_C_H_ */
