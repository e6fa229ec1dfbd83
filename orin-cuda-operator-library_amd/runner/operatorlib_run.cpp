// operatorlib_run: one launcher at a time, with the reference's standalone
// benchmark flags and key=value report lines.
//
// Mirrors the per-operator programs the reference's runner drives
// (tools/run_final_standalone.sh:46-87: reduce_v3 --n=, softmax_v4 --rows=
// --cols= --extreme, transpose_v2 --rows= --cols=, rmsnorm_v3 --tokens=
// --hidden=, gemm --m= --n= --k=, attention --b= --h= --s= --d= --causal=
// --extreme=, each with --warmup= --repeat=) and their output format
// (reduce/reduce_v3.cu:216-226: key=value lines, median time, effective
// bandwidth, correct=PASS/FAIL). Here every operator runs through the C ABI
// of liboperatorlib.so on one HIP stream; the result is checked against an
// fp64 computation on the host (all rows, or a seeded sample of rows for
// GEMM / attention shapes too large to recompute in full).
//
// usage: operatorlib_run <op> [--flag=value ...]
//   ops: reduce softmax transpose rmsnorm gemm_f32 gemm_f16 attention_f32
//        attention_f16
// exit status: 0 when correct=PASS, 1 on FAIL, 2 on usage errors.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iterator>
#include <map>
#include <string>
#include <vector>

#include "operatorlib/operatorlib_c.h"

namespace {

#define RUN_HIP(call)                                                          \
  do {                                                                         \
    const hipError_t run_error_ = (call);                                      \
    if (run_error_ != hipSuccess) {                                            \
      std::fprintf(stderr, "%s:%d %s -> %s\n", __FILE__, __LINE__, #call,      \
                   hipGetErrorString(run_error_));                             \
      std::exit(2);                                                            \
    }                                                                          \
  } while (0)

// ------------------------------------------------------------------ options

struct Options {
  std::map<std::string, std::string> values;

  long long get(const std::string& key, long long fallback) const {
    auto it = values.find(key);
    return it == values.end() ? fallback : std::atoll(it->second.c_str());
  }
  double real(const std::string& key, double fallback) const {
    auto it = values.find(key);
    return it == values.end() ? fallback : std::atof(it->second.c_str());
  }
  bool flag(const std::string& key) const {
    auto it = values.find(key);
    return it != values.end() && it->second != "0" && it->second != "false";
  }
};

Options parse(int argc, char** argv) {
  Options o;
  for (int i = 2; i < argc; ++i) {
    std::string a = argv[i];
    if (a.rfind("--", 0) != 0) {
      std::fprintf(stderr, "unexpected argument: %s\n", argv[i]);
      std::exit(2);
    }
    a = a.substr(2);
    const std::size_t eq = a.find('=');
    if (eq == std::string::npos) o.values[a] = "1";  // bare switch (--extreme)
    else o.values[a.substr(0, eq)] = a.substr(eq + 1);
  }
  return o;
}

// --------------------------------------------------------- inputs, helpers

// xorshift64* stream; uniform values in [lo, hi).
struct Random {
  std::uint64_t s;
  explicit Random(std::uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
  double next() {
    s ^= s >> 12;
    s ^= s << 25;
    s ^= s >> 27;
    return static_cast<double>((s * 0x2545F4914F6CDD1Dull) >> 11) * 0x1.0p-53;
  }
  std::vector<float> uniform(std::size_t n, float lo, float hi) {
    std::vector<float> v(n);
    for (float& x : v) x = static_cast<float>(lo + (hi - lo) * next());
    return v;
  }
};

// fp32 -> binary16 bits, round to nearest even; the host value is replaced by
// the rounded number so the host reference sees what the device does.
std::vector<std::uint16_t> to_half(std::vector<float>& v) {
  std::vector<std::uint16_t> h(v.size());
  for (std::size_t i = 0; i < v.size(); ++i) {
    const _Float16 x = static_cast<_Float16>(v[i]);
    std::memcpy(&h[i], &x, 2);
    v[i] = static_cast<float>(x);
  }
  return h;
}

template <typename T>
T* upload(const std::vector<T>& host) {
  T* d = nullptr;
  RUN_HIP(hipMalloc(&d, std::max<std::size_t>(host.size(), 1) * sizeof(T)));
  RUN_HIP(hipMemcpy(d, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

std::vector<float> download(const float* d, std::size_t n) {
  std::vector<float> h(n);
  RUN_HIP(hipMemcpy(h.data(), d, n * sizeof(float), hipMemcpyDeviceToHost));
  return h;
}

// Median launch time (ms) of `launch` over `repeat` timed launches.
template <typename F>
double median_ms(F launch, int warmup, int repeat, hipStream_t stream) {
  for (int i = 0; i < warmup; ++i) RUN_HIP(static_cast<hipError_t>(launch()));
  RUN_HIP(hipStreamSynchronize(stream));
  hipEvent_t a, b;
  RUN_HIP(hipEventCreate(&a));
  RUN_HIP(hipEventCreate(&b));
  std::vector<double> t;
  for (int i = 0; i < std::max(repeat, 1); ++i) {
    RUN_HIP(hipEventRecord(a, stream));
    RUN_HIP(static_cast<hipError_t>(launch()));
    RUN_HIP(hipEventRecord(b, stream));
    RUN_HIP(hipEventSynchronize(b));
    float ms = 0.0f;
    RUN_HIP(hipEventElapsedTime(&ms, a, b));
    t.push_back(ms);
  }
  RUN_HIP(hipEventDestroy(a));
  RUN_HIP(hipEventDestroy(b));
  std::sort(t.begin(), t.end());
  return t[t.size() / 2];
}

// Rows checked for large shapes: first, last and seeded random ones.
std::vector<long long> sample_rows(long long rows, long long budget, std::uint64_t seed) {
  std::vector<long long> r;
  if (rows <= budget) {
    for (long long i = 0; i < rows; ++i) r.push_back(i);
    return r;
  }
  Random rnd(seed);
  r.push_back(0);
  r.push_back(rows - 1);
  while (static_cast<long long>(r.size()) < budget)
    r.push_back(static_cast<long long>(rnd.next() * rows));
  return r;
}

// How a check's error is measured against its bound.
enum class Bound {
  kRelative,  // max |y - ref| / |ref| over |ref| >= 1e-30
  kAbsolute,  // max |y - ref|
  kMixed,     // max |y - ref| / (1 + |ref|), i.e. |y - ref| <= b + b |ref|
};

struct Report {
  std::string op, shape;
  double ms = 0, bytes = 0, flops = 0, max_abs = 0, max_rel = 0, max_mixed = 0, bound = 0;
  Bound kind = Bound::kRelative;
  long long checked = 0;
};

const char* bound_name(Bound kind) {
  return kind == Bound::kRelative ? "rel" : kind == Bound::kAbsolute ? "abs" : "mixed";
}

double measured(const Report& r) {
  return r.kind == Bound::kRelative ? r.max_rel
         : r.kind == Bound::kAbsolute ? r.max_abs
                                      : r.max_mixed;
}

int finish(const Report& r) {
  hipDeviceProp_t p;
  int dev = 0;
  RUN_HIP(hipGetDevice(&dev));
  RUN_HIP(hipGetDeviceProperties(&p, dev));
  const bool ok = measured(r) <= r.bound && std::isfinite(r.max_abs);
  std::printf("device=%s cu_count=%d\n", p.name, p.multiProcessorCount);
  std::printf("op=%s %s\n", r.op.c_str(), r.shape.c_str());
  std::printf("checked_rows=%lld max_abs_error=%.6e max_rel_error=%.6e", r.checked,
              r.max_abs, r.max_rel);
  if (r.kind == Bound::kMixed) std::printf(" max_mixed_error=%.6e", r.max_mixed);
  std::printf(" %s_bound=%.1e\n", bound_name(r.kind), r.bound);
  std::printf("median_ms=%.6f", r.ms);
  if (r.bytes > 0) std::printf(" effective_bandwidth_GBps=%.3f", r.bytes / (r.ms * 1e6));
  if (r.flops > 0) std::printf(" tflops=%.3f", r.flops / (r.ms * 1e9));
  std::printf("\ncorrect=%s\n", ok ? "PASS" : "FAIL");
  return ok ? 0 : 1;
}

void compare(Report& r, double got, double want) {
  const double err = std::fabs(got - want);
  r.max_abs = std::isnan(got) ? INFINITY : std::max(r.max_abs, err);
  if (std::fabs(want) >= 1e-30) r.max_rel = std::max(r.max_rel, err / std::fabs(want));
  r.max_mixed = std::isnan(got) ? INFINITY : std::max(r.max_mixed, err / (1.0 + std::fabs(want)));
}

// -------------------------------------------------------------- operators

int run_reduce(const Options& o, hipStream_t s, int warmup, int repeat) {
  const long long n = o.get("n", 16777216);
  Random rnd(o.get("seed", 1));
  std::vector<float> x = rnd.uniform(n, -1.0f, 1.0f);
  float* dx = upload(x);
  float* dy = nullptr;
  RUN_HIP(hipMalloc(&dy, sizeof(float)));
  auto launch = [&] { return operatorlib_reduce_sum_f32(dx, dy, n, s); };
  Report r;
  r.op = "reduce_sum_f32";
  r.shape = "n=" + std::to_string(n);
  r.ms = median_ms(launch, warmup, repeat, s);
  r.bytes = 4.0 * n;
  double ref = 0;
  for (float v : x) ref += v;
  compare(r, download(dy, 1)[0], ref);
  r.checked = 1;
  r.bound = 1e-5;
  RUN_HIP(hipFree(dx));
  RUN_HIP(hipFree(dy));
  return finish(r);
}

int run_softmax(const Options& o, hipStream_t s, int warmup, int repeat) {
  const int rows = static_cast<int>(o.get("rows", 4096));
  const int cols = static_cast<int>(o.get("cols", 1024));
  const float range = o.flag("extreme") ? 1000.0f : 3.0f;
  Random rnd(o.get("seed", 2));
  std::vector<float> x = rnd.uniform(static_cast<std::size_t>(rows) * cols, -range, range);
  float* dx = upload(x);
  float* dy = nullptr;
  RUN_HIP(hipMalloc(&dy, x.size() * sizeof(float)));
  auto launch = [&] { return operatorlib_softmax_f32(dx, dy, rows, cols, s); };
  Report r;
  r.op = "softmax_f32";
  r.shape = "rows=" + std::to_string(rows) + " cols=" + std::to_string(cols);
  r.ms = median_ms(launch, warmup, repeat, s);
  r.bytes = 8.0 * rows * cols;
  const std::vector<float> y = download(dy, x.size());
  for (int i = 0; i < rows; ++i) {
    const float* xr = &x[static_cast<std::size_t>(i) * cols];
    float m = xr[0];
    for (int c = 1; c < cols; ++c) m = std::max(m, xr[c]);
    double sum = 0;
    for (int c = 0; c < cols; ++c) sum += std::exp(static_cast<double>(xr[c] - m));
    for (int c = 0; c < cols; ++c)
      compare(r, y[static_cast<std::size_t>(i) * cols + c],
              std::exp(static_cast<double>(xr[c] - m)) / sum);
  }
  r.checked = rows;
  r.bound = 1e-5;
  RUN_HIP(hipFree(dx));
  RUN_HIP(hipFree(dy));
  return finish(r);
}

int run_transpose(const Options& o, hipStream_t s, int warmup, int repeat) {
  const int rows = static_cast<int>(o.get("rows", 4096));
  const int cols = static_cast<int>(o.get("cols", 4096));
  Random rnd(o.get("seed", 3));
  std::vector<float> x = rnd.uniform(static_cast<std::size_t>(rows) * cols, -1.0f, 1.0f);
  float* dx = upload(x);
  float* dy = nullptr;
  RUN_HIP(hipMalloc(&dy, x.size() * sizeof(float)));
  auto launch = [&] { return operatorlib_transpose_f32(dx, dy, rows, cols, s); };
  Report r;
  r.op = "transpose_f32";
  r.shape = "rows=" + std::to_string(rows) + " cols=" + std::to_string(cols);
  r.ms = median_ms(launch, warmup, repeat, s);
  r.bytes = 8.0 * rows * cols;
  const std::vector<float> y = download(dy, x.size());
  long long mismatches = 0;
  for (int i = 0; i < rows; ++i)
    for (int c = 0; c < cols; ++c)
      if (std::memcmp(&y[static_cast<std::size_t>(c) * rows + i],
                      &x[static_cast<std::size_t>(i) * cols + c], 4) != 0)
        ++mismatches;
  r.max_abs = static_cast<double>(mismatches);  // bit-exact: count mismatches
  r.kind = Bound::kAbsolute;
  r.bound = 0;
  r.checked = rows;
  std::printf("mismatches=%lld\n", mismatches);
  RUN_HIP(hipFree(dx));
  RUN_HIP(hipFree(dy));
  return finish(r);
}

int run_rmsnorm(const Options& o, hipStream_t s, int warmup, int repeat) {
  const int tokens = static_cast<int>(o.get("tokens", 2048));
  const int hidden = static_cast<int>(o.get("hidden", 4096));
  const float eps = static_cast<float>(o.real("eps", 1e-5));
  Random rnd(o.get("seed", 4));
  std::vector<float> x = rnd.uniform(static_cast<std::size_t>(tokens) * hidden, -3.0f, 3.0f);
  std::vector<float> w = rnd.uniform(hidden, 0.5f, 1.5f);
  float* dx = upload(x);
  float* dw = upload(w);
  float* dy = nullptr;
  RUN_HIP(hipMalloc(&dy, x.size() * sizeof(float)));
  auto launch = [&] { return operatorlib_rmsnorm_f32(dx, dw, dy, tokens, hidden, eps, s); };
  Report r;
  r.op = "rmsnorm_f32";
  r.shape = "tokens=" + std::to_string(tokens) + " hidden=" + std::to_string(hidden);
  r.ms = median_ms(launch, warmup, repeat, s);
  r.bytes = (2.0 * tokens * hidden + hidden) * 4.0;
  const std::vector<float> y = download(dy, x.size());
  for (int t = 0; t < tokens; ++t) {
    const float* xr = &x[static_cast<std::size_t>(t) * hidden];
    double ss = 0;
    for (int c = 0; c < hidden; ++c) ss += static_cast<double>(xr[c]) * xr[c];
    const double inv = 1.0 / std::sqrt(ss / hidden + eps);
    for (int c = 0; c < hidden; ++c)
      compare(r, y[static_cast<std::size_t>(t) * hidden + c], xr[c] * inv * w[c]);
  }
  r.checked = tokens;
  r.bound = 1e-5;
  RUN_HIP(hipFree(dx));
  RUN_HIP(hipFree(dw));
  RUN_HIP(hipFree(dy));
  return finish(r);
}

int run_gemm(const Options& o, bool half, hipStream_t s, int warmup, int repeat) {
  const int m = static_cast<int>(o.get("m", 4096));
  const int n = static_cast<int>(o.get("n", 4096));
  const int k = static_cast<int>(o.get("k", 4096));
  Random rnd(o.get("seed", 5));
  std::vector<float> a = rnd.uniform(static_cast<std::size_t>(m) * k, -1.0f, 1.0f);
  std::vector<float> b = rnd.uniform(static_cast<std::size_t>(k) * n, -1.0f, 1.0f);
  float* dc = nullptr;
  RUN_HIP(hipMalloc(&dc, static_cast<std::size_t>(m) * n * sizeof(float)));
  void* da = nullptr;
  void* db = nullptr;
  if (half) {
    da = upload(to_half(a));
    db = upload(to_half(b));
  } else {
    da = upload(a);
    db = upload(b);
  }
  auto launch = [&] {
    return half ? operatorlib_gemm_f16(static_cast<const operatorlib_half_t*>(da),
                                       static_cast<const operatorlib_half_t*>(db), dc, m, n, k, s)
                : operatorlib_gemm_f32(static_cast<const float*>(da),
                                       static_cast<const float*>(db), dc, m, n, k, s);
  };
  Report r;
  r.op = half ? "gemm_f16" : "gemm_f32";
  r.shape = "m=" + std::to_string(m) + " n=" + std::to_string(n) + " k=" + std::to_string(k);
  r.ms = median_ms(launch, warmup, repeat, s);
  r.flops = 2.0 * m * n * k;
  const std::vector<float> c = download(dc, static_cast<std::size_t>(m) * n);
  const std::vector<long long> rows =
      sample_rows(m, std::max<long long>(1, (1LL << 28) / (static_cast<long long>(n) * k)), 7);
  double num = 0, den = 0;
  std::vector<double> acc(n);
  for (long long i : rows) {
    std::fill(acc.begin(), acc.end(), 0.0);
    for (int kk = 0; kk < k; ++kk) {
      const double av = a[static_cast<std::size_t>(i) * k + kk];
      const float* br = &b[static_cast<std::size_t>(kk) * n];
      for (int j = 0; j < n; ++j) acc[j] += av * br[j];
    }
    for (int j = 0; j < n; ++j) {
      const double got = c[static_cast<std::size_t>(i) * n + j];
      compare(r, got, acc[j]);
      num += (got - acc[j]) * (got - acc[j]);
      den += acc[j] * acc[j];
    }
  }
  r.checked = static_cast<long long>(rows.size());
  if (half) {  // fp16: max-abs against fp64 on the rounded inputs
    r.kind = Bound::kAbsolute;
    r.bound = 2e-3;
  } else {  // fp32: Frobenius relative error
    r.max_rel = std::sqrt(num / std::max(den, 1e-300));
    r.bound = 1e-4;
  }
  RUN_HIP(hipFree(da));
  RUN_HIP(hipFree(db));
  RUN_HIP(hipFree(dc));
  return finish(r);
}

int run_attention(const Options& o, bool half, hipStream_t s, int warmup, int repeat) {
  const int batch = static_cast<int>(o.get("b", 1));
  const int heads = static_cast<int>(o.get("h", 12));
  const int seq = static_cast<int>(o.get("s", 1024));
  const int d = static_cast<int>(o.get("d", 128));
  const bool causal = o.flag("causal");
  const float range = o.flag("extreme") ? 20.0f : 1.0f;
  const std::size_t count = static_cast<std::size_t>(batch) * heads * seq * d;
  Random rnd(o.get("seed", 6));
  std::vector<float> q = rnd.uniform(count, -range, range);
  std::vector<float> k = rnd.uniform(count, -range, range);
  std::vector<float> v = rnd.uniform(count, -1.0f, 1.0f);
  float* dout = nullptr;
  RUN_HIP(hipMalloc(&dout, count * sizeof(float)));
  void *dq, *dk, *dv;
  if (half) {
    dq = upload(to_half(q));
    dk = upload(to_half(k));
    dv = upload(to_half(v));
  } else {
    dq = upload(q);
    dk = upload(k);
    dv = upload(v);
  }
  auto launch = [&] {
    return half ? operatorlib_attention_f16(
                      static_cast<const operatorlib_half_t*>(dq), static_cast<const operatorlib_half_t*>(dk),
                      static_cast<const operatorlib_half_t*>(dv), dout, batch, heads, seq, d, causal, s)
                : operatorlib_attention_f32(static_cast<const float*>(dq), static_cast<const float*>(dk),
                                            static_cast<const float*>(dv), dout, batch, heads, seq, d,
                                            causal, s);
  };
  Report r;
  r.op = half ? "attention_f16" : "attention_f32";
  r.shape = "b=" + std::to_string(batch) + " h=" + std::to_string(heads) + " s=" +
            std::to_string(seq) + " d=" + std::to_string(d) + " causal=" + (causal ? "1" : "0");
  r.ms = median_ms(launch, warmup, repeat, s);
  // effective (unmasked) flops; the reference counts causal as dense
  r.flops = 4.0 * batch * heads * d * (causal ? seq * (seq + 1.0) / 2.0 : 1.0 * seq * seq);
  const std::vector<float> out = download(dout, count);
  const long long total_rows = static_cast<long long>(batch) * heads * seq;
  const std::vector<long long> rows =
      sample_rows(total_rows, std::max<long long>(1, (1LL << 27) / (2LL * seq * d)), 8);
  const double scale = 1.0 / std::sqrt(static_cast<double>(d));
  std::vector<double> p(seq);
  for (long long g : rows) {
    const long long bh = g / seq;
    const int i = static_cast<int>(g % seq);
    const std::size_t base = static_cast<std::size_t>(bh) * seq * d;
    const int visible = causal ? i + 1 : seq;
    double mx = -INFINITY;
    for (int j = 0; j < visible; ++j) {
      double dot = 0;
      for (int x = 0; x < d; ++x)
        dot += static_cast<double>(q[base + static_cast<std::size_t>(i) * d + x]) *
               k[base + static_cast<std::size_t>(j) * d + x];
      p[j] = dot * scale;
      mx = std::max(mx, p[j]);
    }
    double sum = 0;
    for (int j = 0; j < visible; ++j) sum += (p[j] = std::exp(p[j] - mx));
    for (int x = 0; x < d; ++x) {
      double acc = 0;
      for (int j = 0; j < visible; ++j) acc += p[j] * v[base + static_cast<std::size_t>(j) * d + x];
      compare(r, out[base + static_cast<std::size_t>(i) * d + x], acc / sum);
    }
  }
  r.checked = static_cast<long long>(rows.size());
  // fp16: |y - ref| <= 2e-3 (2e-2 for the +-20 inputs); fp32: |y - ref| <=
  // 1e-4 + 1e-4 |ref| (tests/attention_smoke.cu:108 of the reference).
  r.kind = half ? Bound::kAbsolute : Bound::kMixed;
  r.bound = half ? (o.flag("extreme") ? 2e-2 : 2e-3) : 1e-4;
  RUN_HIP(hipFree(dq));
  RUN_HIP(hipFree(dk));
  RUN_HIP(hipFree(dv));
  RUN_HIP(hipFree(dout));
  return finish(r);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr,
                 "usage: %s reduce|softmax|transpose|rmsnorm|gemm_f32|gemm_f16|"
                 "attention_f32|attention_f16 [--flag=value ...]\n",
                 argv[0]);
    return 2;
  }
  const std::string op = argv[1];
  static const char* const kOps[] = {"reduce",  "softmax",  "transpose",     "rmsnorm",
                                     "gemm_f32", "gemm_f16", "attention_f32", "attention_f16"};
  if (std::find(std::begin(kOps), std::end(kOps), op) == std::end(kOps)) {
    std::fprintf(stderr, "unknown op: %s\n", op.c_str());  // before any HIP call
    return 2;
  }
  const Options o = parse(argc, argv);
  const int warmup = static_cast<int>(o.get("warmup", 10));
  const int repeat = static_cast<int>(o.get("repeat", 30));
  hipStream_t s = nullptr;
  RUN_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  int rc = 2;
  if (op == "reduce") rc = run_reduce(o, s, warmup, repeat);
  else if (op == "softmax") rc = run_softmax(o, s, warmup, repeat);
  else if (op == "transpose") rc = run_transpose(o, s, warmup, repeat);
  else if (op == "rmsnorm") rc = run_rmsnorm(o, s, warmup, repeat);
  else if (op == "gemm_f32") rc = run_gemm(o, false, s, warmup, repeat);
  else if (op == "gemm_f16") rc = run_gemm(o, true, s, warmup, repeat);
  else if (op == "attention_f32") rc = run_attention(o, false, s, warmup, repeat);
  else if (op == "attention_f16") rc = run_attention(o, true, s, warmup, repeat);
  RUN_HIP(hipStreamDestroy(s));
  return rc;
}
