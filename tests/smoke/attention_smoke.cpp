// attention_smoke: attention_f32 / attention_f16 through the C++ API.
//
// The six cases of the reference's tests/attention_smoke.cu:165-177
// (B1 H2; S32 D64 non-causal, S32 D128 causal, S37 D71 causal with
// "extreme" +-20 Q/K), plus shapes on this library's fp16 fast path
// (S % 128 == 0, D 64 / 128). Q and K are U[-r, r] with r = 1 or 20, V is
// U[-1, 1]; fp16 inputs are rounded first and the fp64 oracle sees the
// rounded values (tests/attention_smoke.cu:127-140). Bounds:
// fp32 |y - ref| <= 1e-4 + 1e-4 |ref| (the reference's, :108); fp16
// max-abs 2e-3, or the reference's 2e-2 (:154) for the extreme inputs.
#include "smoke_common.hpp"

namespace {

struct Case {
  int s, d;
  bool causal, extreme;
};

void inputs(const Case& c, std::size_t count, std::vector<float>& q,
            std::vector<float>& k, std::vector<float>& v, std::uint64_t seed) {
  const float r = c.extreme ? 20.0f : 1.0f;
  q = smoke::uniform(seed, count, -r, r);
  k = smoke::uniform(seed + 1, count, -r, r);
  v = smoke::uniform(seed + 2, count, -1.0f, 1.0f);
}

template <typename In>
void run(hipStream_t stream, const Case& c) {
  constexpr int batch = 1, heads = 2;
  const bool half = sizeof(In) == 2;
  const std::size_t count = static_cast<std::size_t>(batch) * heads * c.s * c.d;
  std::vector<float> q, k, v;
  inputs(c, count, q, k, v, (half ? 43 : 31) + c.s + c.d);
  std::vector<In> hq, hk, hv;
  if constexpr (sizeof(In) == 2) {
    hq = smoke::to_half(q);
    hk = smoke::to_half(k);
    hv = smoke::to_half(v);
  } else {
    hq = q;
    hk = k;
    hv = v;
  }
  smoke::DeviceArray<In> dq(hq, stream), dk(hk, stream), dv(hv, stream);
  smoke::DeviceArray<float> out(count);
  if constexpr (sizeof(In) == 2)
    SMOKE_HIP(operatorlib::attention_f16(dq.get(), dk.get(), dv.get(), out.get(), batch,
                                         heads, c.s, c.d, c.causal, stream));
  else
    SMOKE_HIP(operatorlib::attention_f32(dq.get(), dk.get(), dv.get(), out.get(), batch,
                                         heads, c.s, c.d, c.causal, stream));
  const std::vector<float> got = out.download(stream);
  std::vector<double> want(count);
  oracle_attention(q.data(), k.data(), v.data(), want.data(), batch * heads, c.s, c.d,
                   c.causal, nullptr, nullptr, 0);
  bool ok = true;
  double worst = 0.0;
  const double bound = half ? (c.extreme ? 2e-2 : 2e-3) : 1e-4;
  for (std::size_t i = 0; i < count; ++i) {
    const double err = std::abs(got[i] - want[i]);
    worst = std::max(worst, err);
    const double allowed = half ? bound : 1e-4 + 1e-4 * std::abs(want[i]);
    if (!std::isfinite(got[i]) || err > allowed) ok = false;
  }
  char name[96];
  std::snprintf(name, sizeof name, "attention_%s[S%d,D%d,causal%d,extreme%d]",
                half ? "f16" : "f32", c.s, c.d, c.causal ? 1 : 0, c.extreme ? 1 : 0);
  smoke::report(name, ok, worst, bound);
}

}  // namespace

int main() {
  hipStream_t stream = nullptr;
  SMOKE_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
  const Case reference_cases[] = {{32, 64, false, false}, {32, 128, true, false},
                                  {37, 71, true, true}};
  for (const Case& c : reference_cases) run<float>(stream, c);
  for (const Case& c : reference_cases) run<__half>(stream, c);
  const Case fast_path[] = {{128, 128, true, false}, {256, 64, false, false},
                            {384, 128, true, false}};
  for (const Case& c : fast_path) run<__half>(stream, c);
  SMOKE_HIP(hipStreamDestroy(stream));
  return smoke::finish("attention_smoke");
}
