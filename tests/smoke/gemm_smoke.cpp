// gemm_smoke: gemm_f32 / gemm_f16 through the C++ API at the dispatch shapes
// of the reference's tests/gemm_smoke.cu:141-148 (its M = 1, M <= 16,
// tiled and ragged cases), plus shapes that take this library's fp16
// global-to-LDS fast path and its ragged fallback.
//
// The reference compares against cuBLAS with a mixed 2e-2 bound; here the
// expected values are the fp64 oracle on the same (fp16-rounded) inputs and
// the bounds are this library's: fp32 Frobenius rel 1e-4, fp16 max-abs 2e-3.
#include "smoke_common.hpp"

namespace {

double frobenius_rel(const std::vector<float>& got, const std::vector<double>& want) {
  double num = 0.0, den = 0.0;
  for (std::size_t i = 0; i < got.size(); ++i) {
    if (!std::isfinite(got[i])) return INFINITY;
    num += (got[i] - want[i]) * (got[i] - want[i]);
    den += want[i] * want[i];
  }
  return std::sqrt(num / den);
}

double max_abs(const std::vector<float>& got, const std::vector<double>& want) {
  double worst = 0.0;
  for (std::size_t i = 0; i < got.size(); ++i) {
    if (!std::isfinite(got[i])) return INFINITY;
    worst = std::max(worst, std::abs(got[i] - want[i]));
  }
  return worst;
}

void f32_case(hipStream_t stream, int m, int n, int k) {
  std::vector<float> a = smoke::uniform(17 + m, static_cast<std::size_t>(m) * k, -0.25f, 0.25f);
  std::vector<float> b = smoke::uniform(18 + n, static_cast<std::size_t>(k) * n, -0.25f, 0.25f);
  smoke::DeviceArray<float> da(a, stream), db(b, stream), dc(static_cast<std::size_t>(m) * n);
  SMOKE_HIP(operatorlib::gemm_f32(da.get(), db.get(), dc.get(), m, n, k, stream));
  const std::vector<float> got = dc.download(stream);
  std::vector<double> want(got.size());
  oracle_gemm(a.data(), b.data(), want.data(), m, n, k, nullptr, 0);
  const double err = frobenius_rel(got, want);
  char name[64];
  std::snprintf(name, sizeof name, "gemm_f32[%d,%d,%d]", m, n, k);
  smoke::report(name, err <= 1e-4, err, 1e-4);
}

void f16_case(hipStream_t stream, int m, int n, int k) {
  std::vector<float> a = smoke::uniform(19 + m, static_cast<std::size_t>(m) * k, -0.25f, 0.25f);
  std::vector<float> b = smoke::uniform(20 + n, static_cast<std::size_t>(k) * n, -0.25f, 0.25f);
  const std::vector<__half> ha = smoke::to_half(a), hb = smoke::to_half(b);
  smoke::DeviceArray<__half> da(ha, stream), db(hb, stream);
  smoke::DeviceArray<float> dc(static_cast<std::size_t>(m) * n);
  SMOKE_HIP(operatorlib::gemm_f16(da.get(), db.get(), dc.get(), m, n, k, stream));
  const std::vector<float> got = dc.download(stream);
  std::vector<double> want(got.size());
  oracle_gemm(a.data(), b.data(), want.data(), m, n, k, nullptr, 0);
  const double err = max_abs(got, want);
  char name[64];
  std::snprintf(name, sizeof name, "gemm_f16[%d,%d,%d]", m, n, k);
  smoke::report(name, err <= 2e-3, err, 2e-3);
}

}  // namespace

int main() {
  hipStream_t stream = nullptr;
  SMOKE_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  f32_case(stream, 1, 256, 64);
  f32_case(stream, 16, 128, 64);
  f32_case(stream, 128, 64, 32);
  f32_case(stream, 37, 65, 71);
  f16_case(stream, 128, 128, 32);
  f16_case(stream, 16, 128, 32);
  f16_case(stream, 32, 32, 32);
  f16_case(stream, 37, 65, 71);
  f16_case(stream, 1, 4096, 4096);   // decode-shaped, fast path
  f16_case(stream, 300, 520, 192);   // fast path, ragged M and N tiles
  f16_case(stream, 513, 136, 1000);  // K not a multiple of 64: fallback
  SMOKE_HIP(hipStreamDestroy(stream));
  return smoke::finish("gemm_smoke");
}
