/*
 * operatorlib CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU reference computations, used
 * by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker. The library never links, loads or calls it.
 *
 * Each function cites the reference code it follows. All accumulation is in
 * fp64, as in the reference; functions return fp64 results so callers can
 * measure error against the exact-as-possible value (the reference rounds
 * to fp32 at the end; oracle.py offers both).
 *
 * The seeded generator is defined here (the reference's std::mt19937 +
 * std::uniform_real_distribution output is implementation-defined, so its
 * inputs are not portable): SplitMix64, uniform by exact 24-bit mapping,
 * normal by Box-Muller in fp64 (cosine branch only).
 */
#ifndef OPERATORLIB_ORACLE_H_
#define OPERATORLIB_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* --- generator ----------------------------------------------------------- */
uint64_t oracle_splitmix64(uint64_t* state);
/* out[i] = lo + (hi - lo) * u_i, u_i = (x_i >> 40) * 2^-24 in [0, 1). */
void oracle_fill_uniform(uint64_t seed, float lo, float hi, float* out,
                         size_t n);
/* out[i] = mean + stddev * sqrt(-2 ln u1) cos(2 pi u2), u1 in (0,1], u2 in
 * [0,1), both with 53-bit resolution, two SplitMix64 draws per value. */
void oracle_fill_normal(uint64_t seed, float mean, float stddev, float* out,
                        size_t n);

/* --- fp16 ----------------------------------------------------------------- */
/* IEEE binary16 round-to-nearest-even (the rounding of __float2half_rn,
 * reference attention/attention_v6.cu:23-30). */
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
void oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* --- operators ------------------------------------------------------------ */
/* reduce/reduce_v3.cu:125-128: sequential fp64 accumulation. */
double oracle_reduce_sum(const float* input, size_t n);

/* softmax/softmax_v4.cu:253-268: fp32 row max, exp(float(x - max)) in fp64,
 * fp64 sum, fp64 divide. */
void oracle_softmax(const float* input, double* output, int rows, int cols);

/* transpose/transpose_v2.cu:104-113. */
void oracle_transpose(const float* input, float* output, int rows, int cols);

/* rmsnorm/rmsnorm_v3.cu:154-172: fp64 sum of squares,
 * 1 / sqrt(ss / hidden + eps), x * inv * w in fp64. */
void oracle_rmsnorm(const float* input, const float* weight, double* output,
                    int tokens, int hidden, float epsilon);

/* Textbook fp64 C = A B (row-major). The reference has no CPU GEMM (it uses
 * cuBLAS, gemm/gemm_common.h:80-86); this is the fp64 ground truth it is
 * judged against. Computes only the listed rows (rows == NULL: all m rows,
 * in order); output row r of `c` holds C[rows[r], :]. */
void oracle_gemm(const float* a, const float* b, double* c, int m, int n,
                 int k, const int* rows, int nrows);

/* attention/attention_common.h:123-156 (= tests/attention_smoke.cu:31-66):
 * fp64 scores scaled by 1/sqrt(d), causal keys j <= i, fp64 softmax and PV.
 * Tensors are [bh][s][d]. Computes only the listed (head, row) pairs
 * (heads/rows NULL: every row of every head, in order); output entry r of
 * `out` holds d values. */
void oracle_attention(const float* q, const float* k, const float* v,
                      double* out, int bh, int s, int d, int causal,
                      const int* heads, const int* rows, int nrows);

#ifdef __cplusplus
}
#endif

#endif /* OPERATORLIB_ORACLE_H_ */
