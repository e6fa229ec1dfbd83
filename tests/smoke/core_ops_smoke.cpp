// core_ops_smoke: reduce, softmax, transpose and RMSNorm through the C++ API
// (plus the FP16 softmax / RMSNorm launchers this library adds).
//
// Same cases as the reference's tests/core_ops_smoke.cu:165-180 (iota
// reduce, softmax 19x128 / 17x1024 at range 5 and 17x1003 at range 1000,
// a 37x65 iota transpose, RMSNorm 32x4096 and 17x1003 with eps 1e-5), on a
// non-blocking stream, with this library's tolerances: reduce rel 1e-5
// (the iota sum -500 must come out exact), softmax / RMSNorm elementwise
// rel 1e-5, transpose bit-exact.
#include <numeric>

#include "smoke_common.hpp"

namespace {

void reduce_iota(hipStream_t stream) {
  std::vector<float> x(1000);
  std::iota(x.begin(), x.end(), -500.0f);
  smoke::DeviceArray<float> in(x, stream), out(1);
  SMOKE_HIP(operatorlib::reduce_sum_f32(in.get(), out.get(), x.size(), stream));
  const float got = out.download(stream)[0];
  const double want = oracle_reduce_sum(x.data(), x.size());
  smoke::report("reduce_sum_f32[iota1000]", got == -500.0f && want == -500.0,
                std::abs(got - want), 0.0);
}

void reduce_random(hipStream_t stream, std::size_t n) {
  std::vector<float> x = smoke::uniform(41 + n, n, -1.0f, 1.0f);
  smoke::DeviceArray<float> in(x, stream), out(1);
  SMOKE_HIP(operatorlib::reduce_sum_f32(in.get(), out.get(), n, stream));
  const double got = out.download(stream)[0];
  const double want = oracle_reduce_sum(x.data(), n);
  const double err = std::abs(got - want);
  char name[64];
  std::snprintf(name, sizeof name, "reduce_sum_f32[%zu]", n);
  smoke::report(name, err <= 1e-5 * std::abs(want), err, 1e-5 * std::abs(want));
}

void softmax_case(hipStream_t stream, int rows, int cols, float range) {
  const std::size_t count = static_cast<std::size_t>(rows) * cols;
  std::vector<float> x = smoke::uniform(7 + rows + cols, count, -range, range);
  smoke::DeviceArray<float> in(x, stream), out(count);
  SMOKE_HIP(operatorlib::softmax_f32(in.get(), out.get(), rows, cols, stream));
  const std::vector<float> got = out.download(stream);
  std::vector<double> want(count);
  oracle_softmax(x.data(), want.data(), rows, cols);
  double worst = 0.0, worst_row_sum = 0.0;
  for (int r = 0; r < rows; ++r) {
    double row_sum = 0.0;
    for (int c = 0; c < cols; ++c) {
      const std::size_t i = static_cast<std::size_t>(r) * cols + c;
      row_sum += got[i];
      if (std::abs(want[i]) >= 1e-30 && std::isfinite(got[i]))
        worst = std::max(worst, std::abs(got[i] - want[i]) / std::abs(want[i]));
      else if (!std::isfinite(got[i]))
        worst = INFINITY;
    }
    worst_row_sum = std::max(worst_row_sum, std::abs(row_sum - 1.0));
  }
  char name[64];
  std::snprintf(name, sizeof name, "softmax_f32[%dx%d,range%g]", rows, cols, range);
  smoke::report(name, worst <= 1e-5 && worst_row_sum <= 1e-5, worst, 1e-5);
}

void transpose_iota(hipStream_t stream) {
  constexpr int rows = 37, cols = 65;
  std::vector<float> x(rows * cols);
  std::iota(x.begin(), x.end(), -100.0f);
  smoke::DeviceArray<float> in(x, stream), out(x.size());
  SMOKE_HIP(operatorlib::transpose_f32(in.get(), out.get(), rows, cols, stream));
  const std::vector<float> got = out.download(stream);
  std::vector<float> want(x.size());
  oracle_transpose(x.data(), want.data(), rows, cols);
  const bool same = std::memcmp(got.data(), want.data(), x.size() * sizeof(float)) == 0;
  smoke::report("transpose_f32[37x65]", same, same ? 0.0 : 1.0, 0.0);
}

void rmsnorm_case(hipStream_t stream, int tokens, int hidden) {
  constexpr float eps = 1.0e-5f;
  const std::size_t count = static_cast<std::size_t>(tokens) * hidden;
  std::vector<float> x = smoke::uniform(11 + tokens, count, -3.0f, 3.0f);
  std::vector<float> w = smoke::uniform(12 + hidden, hidden, 0.5f, 1.5f);
  smoke::DeviceArray<float> in(x, stream), weight(w, stream), out(count);
  SMOKE_HIP(operatorlib::rmsnorm_f32(in.get(), weight.get(), out.get(), tokens,
                                     hidden, eps, stream));
  const std::vector<float> got = out.download(stream);
  std::vector<double> want(count);
  oracle_rmsnorm(x.data(), w.data(), want.data(), tokens, hidden, eps);
  double worst = 0.0;
  for (std::size_t i = 0; i < count; ++i) {
    if (!std::isfinite(got[i])) { worst = INFINITY; break; }
    if (std::abs(want[i]) >= 1e-30)
      worst = std::max(worst, std::abs(got[i] - want[i]) / std::abs(want[i]));
  }
  char name[64];
  std::snprintf(name, sizeof name, "rmsnorm_f32[%dx%d]", tokens, hidden);
  smoke::report(name, worst <= 1e-5, worst, 1e-5);
}

// FP16 rows (softmax_f16 / rmsnorm_f16, not in the reference API): fp16 in
// and out, fp32 arithmetic; each output within one fp16 ulp of the fp64
// oracle on the same fp16 inputs (|y - ref| <= 2^-10 |ref| + 2^-24).
double f16_error(const std::vector<__half>& got, const std::vector<double>& want) {
  std::vector<std::uint16_t> bits(got.size());
  std::memcpy(bits.data(), got.data(), bits.size() * sizeof(std::uint16_t));
  std::vector<float> y(got.size());
  oracle_f16_to_f32_array(bits.data(), y.data(), y.size());
  double worst = 0.0;  // in units of the bound
  for (std::size_t i = 0; i < y.size(); ++i) {
    if (!std::isfinite(y[i])) return INFINITY;
    const double bound = std::ldexp(std::abs(want[i]), -10) + std::ldexp(1.0, -24);
    worst = std::max(worst, std::abs(y[i] - want[i]) / bound);
  }
  return worst;
}

void softmax_f16_case(hipStream_t stream, int rows, int cols, float range) {
  const std::size_t count = static_cast<std::size_t>(rows) * cols;
  std::vector<float> x = smoke::uniform(21 + rows + cols, count, -range, range);
  const std::vector<__half> hx = smoke::to_half(x);  // x now holds the fp16 values
  smoke::DeviceArray<__half> in(hx, stream), out(count);
  SMOKE_HIP(operatorlib::softmax_f16(in.get(), out.get(), rows, cols, stream));
  std::vector<double> want(count);
  oracle_softmax(x.data(), want.data(), rows, cols);
  const double worst = f16_error(out.download(stream), want);
  char name[64];
  std::snprintf(name, sizeof name, "softmax_f16[%dx%d,range%g]", rows, cols, range);
  smoke::report(name, worst <= 1.0, worst, 1.0);
}

void rmsnorm_f16_case(hipStream_t stream, int tokens, int hidden) {
  constexpr float eps = 1.0e-5f;
  const std::size_t count = static_cast<std::size_t>(tokens) * hidden;
  std::vector<float> x = smoke::uniform(31 + tokens, count, -3.0f, 3.0f);
  std::vector<float> w = smoke::uniform(32 + hidden, hidden, 0.5f, 1.5f);
  const std::vector<__half> hx = smoke::to_half(x), hw = smoke::to_half(w);
  smoke::DeviceArray<__half> in(hx, stream), weight(hw, stream), out(count);
  SMOKE_HIP(operatorlib::rmsnorm_f16(in.get(), weight.get(), out.get(), tokens,
                                     hidden, eps, stream));
  std::vector<double> want(count);
  oracle_rmsnorm(x.data(), w.data(), want.data(), tokens, hidden, eps);
  const double worst = f16_error(out.download(stream), want);
  char name[64];
  std::snprintf(name, sizeof name, "rmsnorm_f16[%dx%d]", tokens, hidden);
  smoke::report(name, worst <= 1.0, worst, 1.0);
}

void rejects_invalid_arguments(hipStream_t stream) {
  float* p = reinterpret_cast<float*>(0x1000);  // never dereferenced
  const bool ok =
      operatorlib::reduce_sum_f32(nullptr, p, 4, stream) == hipErrorInvalidValue &&
      operatorlib::softmax_f32(p, p, 0, 4, stream) == hipErrorInvalidValue &&
      operatorlib::transpose_f32(p, p, 4, -1, stream) == hipErrorInvalidValue &&
      operatorlib::rmsnorm_f32(p, p, p, 2, 4, 0.0f, stream) == hipErrorInvalidValue;
  smoke::report("invalid_arguments", ok, ok ? 0.0 : 1.0, 0.0);
}

}  // namespace

int main() {
  hipStream_t stream = nullptr;
  SMOKE_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  reduce_iota(stream);
  reduce_random(stream, 1000003);
  softmax_case(stream, 19, 128, 5.0f);
  softmax_case(stream, 17, 1024, 5.0f);
  softmax_case(stream, 17, 1003, 1000.0f);
  transpose_iota(stream);
  rmsnorm_case(stream, 32, 4096);
  rmsnorm_case(stream, 17, 1003);
  softmax_f16_case(stream, 19, 128, 5.0f);
  softmax_f16_case(stream, 17, 1003, 5.0f);
  rmsnorm_f16_case(stream, 32, 4096);
  rmsnorm_f16_case(stream, 17, 1003);
  rejects_invalid_arguments(stream);
  SMOKE_HIP(hipStreamDestroy(stream));
  return smoke::finish("core_ops_smoke");
}
