// Argument predicates of the C ABI (csrc/validate.hpp), run on the host at
// boundary values. Built with AddressSanitizer and UndefinedBehaviorSanitizer
// (-fno-sanitize-recover), so undefined behaviour that executes (an
// out-of-range read, a signed overflow the compiler keeps) aborts the
// program. The expectations catch predicates that answer wrongly: a 32-bit
// batch * heads product, for instance, which the compiler may fold away
// (int <= INT_MAX is always true) before UBSan sees it. Prints "failures=N";
// exit status 0 only when every expectation holds.
//
// The expected results restate the reference launchers' prologues
// (src/reduce.cu:56-57, src/softmax.cu:184-185, src/transpose.cu:40-41,
// src/rmsnorm.cu:80-82, src/gemm.cu:443-445, src/attention.cu:448-451) plus
// the batch * heads <= INT_MAX bound of its binding
// (python/operatorlib_binding.cpp:164-166).

#include <climits>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <limits>

#include "validate.hpp"

namespace {

int failures = 0;

void expect(bool got, bool want, const char* what, long long a, long long b) {
  if (got != want) {
    std::printf("FAIL %s (%lld, %lld): got %d want %d\n", what, a, b, got, want);
    ++failures;
  }
}

}  // namespace

int main() {
  char storage[16];
  const void* p = storage;
  const int ints[] = {INT_MIN, INT_MIN + 1, -4096, -1, 0, 1, 2, 127, 128, 129,
                      4095, 4096, 46340, 46341, 65536, INT_MAX - 1, INT_MAX};

  for (const int r : ints)
    for (const int c : ints) {
      expect(opl::matrix_args_ok(p, p, r, c), r > 0 && c > 0, "matrix", r, c);
      expect(opl::gemm_args_ok(p, p, p, r, c, 1), r > 0 && c > 0, "gemm m,n", r, c);
      expect(opl::gemm_args_ok(p, p, p, 1, r, c), r > 0 && c > 0, "gemm n,k", r, c);
      expect(opl::rmsnorm_args_ok(p, p, p, r, c, 1e-6f), r > 0 && c > 0, "rmsnorm", r, c);
      // batch * heads must fit int32 (computed in 64 bits: no overflow).
      const bool bh_fits = r > 0 && c > 0 &&
                           static_cast<long long>(r) * c <= INT_MAX;
      expect(opl::attention_args_ok(p, p, p, p, r, c, 1024, 128), bh_fits,
             "attention batch,heads", r, c);
      expect(opl::attention_args_ok(p, p, p, p, 1, 1, r, c),
             r > 0 && c > 0 && c <= opl::kMaxHeadDim, "attention seq,dim", r, c);
    }

  // Null pointers, one at a time.
  expect(opl::matrix_args_ok(nullptr, p, 1, 1), false, "matrix null in", 0, 0);
  expect(opl::matrix_args_ok(p, nullptr, 1, 1), false, "matrix null out", 0, 0);
  expect(opl::reduce_args_ok(nullptr, p, 1), false, "reduce null in", 0, 0);
  expect(opl::reduce_args_ok(p, nullptr, 1), false, "reduce null out", 0, 0);
  expect(opl::rmsnorm_args_ok(p, nullptr, p, 1, 1, 1e-6f), false, "rmsnorm null w", 0, 0);
  expect(opl::gemm_args_ok(p, p, nullptr, 1, 1, 1), false, "gemm null c", 0, 0);
  for (int which = 0; which < 4; ++which) {
    const void* q[4] = {p, p, p, p};
    q[which] = nullptr;
    expect(opl::attention_args_ok(q[0], q[1], q[2], q[3], 1, 1, 1, 1), false,
           "attention null", which, 0);
  }

  // reduce: any n > 0, including the largest size_t.
  const std::size_t sizes[] = {0, 1, 1000003, std::numeric_limits<std::size_t>::max()};
  for (const std::size_t n : sizes)
    expect(opl::reduce_args_ok(p, p, n), n != 0, "reduce n", static_cast<long long>(n % LLONG_MAX), 0);

  // epsilon: the reference's `epsilon <= 0.0f` rejection test
  // (src/rmsnorm.cu:80-81): zero, -0.0 and negatives are rejected; NaN
  // compares false there, so it is accepted, as is +inf.
  const float nan = std::numeric_limits<float>::quiet_NaN();
  const float eps[] = {nan, -nan, -1.0f, -0.0f, 0.0f,
                       std::numeric_limits<float>::denorm_min(), 1e-6f,
                       std::numeric_limits<float>::infinity()};
  const bool eps_ok[] = {true, true, false, false, false, true, true, true};
  for (int i = 0; i < 8; ++i)
    expect(opl::rmsnorm_args_ok(p, p, p, 2, 2, eps[i]), eps_ok[i], "rmsnorm eps", i, 0);

  std::printf("failures=%d\n", failures);
  return failures == 0 ? 0 : 1;
}
