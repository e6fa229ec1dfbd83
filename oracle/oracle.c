/*
 * operatorlib CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this code; the library never does.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- generator */

uint64_t oracle_splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void oracle_fill_uniform(uint64_t seed, float lo, float hi, float* out,
                         size_t n) {
  uint64_t state = seed;
  const double span = (double)hi - (double)lo;
  for (size_t i = 0; i < n; ++i) {
    const double u = (double)(oracle_splitmix64(&state) >> 40) * 0x1p-24;
    out[i] = (float)((double)lo + span * u);
  }
}

void oracle_fill_normal(uint64_t seed, float mean, float stddev, float* out,
                        size_t n) {
  uint64_t state = seed;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; ++i) {
    const double u1 =
        (double)((oracle_splitmix64(&state) >> 11) + 1) * 0x1p-53; /* (0,1] */
    const double u2 = (double)(oracle_splitmix64(&state) >> 11) * 0x1p-53;
    const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    out[i] = (float)((double)mean + (double)stddev * z);
  }
}

/* --------------------------------------------------------------------- fp16 */

uint16_t oracle_f32_to_f16(float x) {
  uint32_t f;
  memcpy(&f, &x, sizeof f);
  const uint16_t sign = (uint16_t)((f >> 16) & 0x8000u);
  const uint32_t exp = (f >> 23) & 0xffu;
  const uint32_t mant = f & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | (mant ? 0x7e00u : 0x7c00u));
  const int e = (int)exp - 127;
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) { /* half normal range; rounding may carry into inf */
    uint32_t h = ((uint32_t)(e + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
  }
  if (exp == 0) return sign; /* fp32 zero or subnormal: far below 2^-25 */
  const int shift = -(e + 1); /* value / 2^-24 = sig * 2^-shift, shift >= 14 */
  if (shift > 24) return sign;
  const uint32_t sig = mant | 0x800000u;
  uint32_t m = sig >> shift;
  const uint32_t rem = sig & ((1u << shift) - 1u);
  const uint32_t halfway = 1u << (shift - 1);
  if (rem > halfway || (rem == halfway && (m & 1u))) m += 1u;
  return (uint16_t)(sign | m);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t mant = h & 0x3ffu;
  uint32_t f;
  if (exp == 0) {
    if (mant == 0) {
      f = sign;
    } else { /* subnormal: mant * 2^-24, exact in fp32 */
      const float v = (float)mant * 0x1p-24f;
      memcpy(&f, &v, sizeof f);
      f |= sign;
    }
  } else if (exp == 0x1fu) {
    f = sign | 0x7f800000u | (mant << 13);
  } else {
    f = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float out;
  memcpy(&out, &f, sizeof out);
  return out;
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

/* ---------------------------------------------------------------- operators */

double oracle_reduce_sum(const float* input, size_t n) {
  double sum = 0.0;
  for (size_t i = 0; i < n; ++i) sum += (double)input[i];
  return sum;
}

void oracle_softmax(const float* input, double* output, int rows, int cols) {
  for (int row = 0; row < rows; ++row) {
    const float* x = input + (size_t)row * cols;
    double* y = output + (size_t)row * cols;
    float maximum = -FLT_MAX;
    for (int c = 0; c < cols; ++c) maximum = x[c] > maximum ? x[c] : maximum;
    double sum = 0.0;
    for (int c = 0; c < cols; ++c) {
      const float shifted = x[c] - maximum; /* fp32 subtraction, as reference */
      sum += exp((double)shifted);
    }
    for (int c = 0; c < cols; ++c) {
      const float shifted = x[c] - maximum;
      y[c] = exp((double)shifted) / sum;
    }
  }
}

void oracle_transpose(const float* input, float* output, int rows, int cols) {
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c)
      output[(size_t)c * rows + r] = input[(size_t)r * cols + c];
}

void oracle_rmsnorm(const float* input, const float* weight, double* output,
                    int tokens, int hidden, float epsilon) {
  for (int t = 0; t < tokens; ++t) {
    const float* x = input + (size_t)t * hidden;
    double* y = output + (size_t)t * hidden;
    double square_sum = 0.0;
    for (int c = 0; c < hidden; ++c) square_sum += (double)x[c] * (double)x[c];
    const double inverse_rms =
        1.0 / sqrt(square_sum / hidden + (double)epsilon);
    for (int c = 0; c < hidden; ++c)
      y[c] = (double)x[c] * inverse_rms * (double)weight[c];
  }
}

void oracle_gemm(const float* a, const float* b, double* c, int m, int n,
                 int k, const int* rows, int nrows) {
  if (rows == NULL) nrows = m;
  for (int r = 0; r < nrows; ++r) {
    const int row = rows ? rows[r] : r;
    double* out = c + (size_t)r * n;
    for (int j = 0; j < n; ++j) out[j] = 0.0;
    const float* arow = a + (size_t)row * k;
    for (int kk = 0; kk < k; ++kk) {
      const double av = (double)arow[kk];
      const float* brow = b + (size_t)kk * n;
      for (int j = 0; j < n; ++j) out[j] += av * (double)brow[j];
    }
  }
}

void oracle_attention(const float* q, const float* k, const float* v,
                      double* out, int bh, int s, int d, int causal,
                      const int* heads, const int* rows, int nrows) {
  const double scale = 1.0 / sqrt((double)d);
  double* scores = (double*)malloc(sizeof(double) * (size_t)s);
  if (scores == NULL) return;
  if (heads == NULL || rows == NULL) nrows = bh * s;
  for (int r = 0; r < nrows; ++r) {
    const int head = heads ? heads[r] : r / s;
    const int row = rows ? rows[r] : r % s;
    const size_t base = (size_t)head * s * d;
    const int visible = causal ? row + 1 : s;
    double maximum = -INFINITY;
    for (int col = 0; col < visible; ++col) {
      double dot = 0.0;
      for (int x = 0; x < d; ++x)
        dot += (double)q[base + (size_t)row * d + x] *
               (double)k[base + (size_t)col * d + x];
      scores[col] = dot * scale;
      if (scores[col] > maximum) maximum = scores[col];
    }
    double denominator = 0.0;
    for (int col = 0; col < visible; ++col) {
      scores[col] = exp(scores[col] - maximum);
      denominator += scores[col];
    }
    double* o = out + (size_t)r * d;
    for (int x = 0; x < d; ++x) {
      double value = 0.0;
      for (int col = 0; col < visible; ++col)
        value += scores[col] * (double)v[base + (size_t)col * d + x];
      o[x] = value / denominator;
    }
  }
  free(scores);
}
