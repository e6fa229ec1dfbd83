// torch.ops.operatorlib.* over the C ABI (operatorlib/operatorlib_c.h).
//
// Drop-in for the reference's python/operatorlib_binding.cpp: the same six
// schema strings (:190-197) registered on the CUDA dispatch key (:199-206),
// which is where PyTorch-ROCm keeps HIP tensors; the same output shapes and
// dtypes (0-d reduce, input-shaped softmax / rmsnorm, [cols, rows]
// transpose, fp32 GEMM and attention outputs); work enqueued on the current
// stream of the inputs' device, never copied, never synchronized. Error
// texts contain the substrings the reference's tests assert
// (python/test_extension.py:124-168): "float32", "contiguous",
// "positive int32", "2D", "weight length", "a.size(1)", "at most 128", and
// "<op> launch failed: " for launch errors.
//
// Structure: an Operands object checks what every operator requires of its
// tensors (HIP device memory on one device, dense row-major, one dtype from
// the operator's set); extent() turns a tensor size into the int the C ABI
// takes; launch() runs one C ABI call under a device guard on the current
// stream. Each operator then states only its own shape rules. Operators
// whose kernels may need scratch (reduce_sum, gemm, attention) call the
// *_ws entry points with a Workspace from torch's allocator.

#include <ATen/ATen.h>
#include <ATen/hip/HIPContext.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <limits>
#include <string>
#include <utility>
#include <vector>

#include "operatorlib/operatorlib_c.h"

namespace {

enum DTypes { kFloat32Only, kFloat32OrFloat16 };

const char* dtype_set_text(DTypes set) {
  return set == kFloat32Only ? "float32" : "float32 or float16";
}

class Operands {
 public:
  // `named` lists (tensor, argument name); the first tensor sets the device
  // and dtype the others must share.
  Operands(const char* op, DTypes allowed,
           std::initializer_list<std::pair<const at::Tensor*, const char*>> named)
      : op_(op), list_(named) {
    const at::Tensor& lead = *list_.front().first;
    for (const auto& [t, name] : list_) {
      TORCH_CHECK(t->is_cuda(), op_, ": ", name,
                  " must live in HIP device memory (a CUDA-key tensor), got ",
                  t->device());
      TORCH_CHECK(t->is_contiguous(), op_, ": ", name,
                  " must be contiguous (dense row-major)");
      TORCH_CHECK(t->device() == lead.device(), op_, ": ", name, " is on ",
                  t->device(), " but ", list_.front().second, " is on ", lead.device());
      TORCH_CHECK(t->scalar_type() == lead.scalar_type(), op_, ": ", name,
                  " has dtype ", t->scalar_type(), " but ", list_.front().second,
                  " has dtype ", lead.scalar_type());
    }
    const at::ScalarType dt = lead.scalar_type();
    const bool ok = dt == at::kFloat || (allowed == kFloat32OrFloat16 && dt == at::kHalf);
    TORCH_CHECK(ok, op_, ": inputs must be ", dtype_set_text(allowed), ", got ", dt);
    half_ = dt == at::kHalf;
  }

  bool half() const { return half_; }
  const at::Tensor& lead() const { return *list_.front().first; }
  const char* op() const { return op_; }

 private:
  const char* op_;
  std::vector<std::pair<const at::Tensor*, const char*>> list_;
  bool half_ = false;
};

// A size the C ABI takes as int: positive and within int32.
int extent(const char* op, const char* what, std::int64_t value) {
  TORCH_CHECK(value > 0 && value <= std::numeric_limits<int>::max(), op, ": ",
              what, " = ", value, " is not a positive int32");
  return static_cast<int>(value);
}

void require_rank(const Operands& in, const at::Tensor& t, const char* name,
                  std::int64_t rank, const char* layout) {
  TORCH_CHECK(t.dim() == rank, in.op(), ": ", name, " must be ", layout, ", got ",
              t.dim(), " dimension(s)");
}

// Rows of a tensor read as [rows, size(-1)].
std::pair<int, int> rows_by_last(const Operands& in, const at::Tensor& t,
                                 const char* last_name) {
  TORCH_CHECK(t.dim() >= 1, in.op(), ": ", "input must have at least one dimension");
  const int last = extent(in.op(), last_name, t.size(-1));
  const int rows = extent(in.op(), "row count (numel / size(-1))", t.numel() / t.size(-1));
  return {rows, last};
}

const void* caddr(const at::Tensor& t) { return t.data_ptr(); }

// Scratch for a *_ws entry point: `bytes` from torch's caching allocator on
// the inputs' device, handed back to it when the operator returns. The
// allocator is stream-ordered (the block is reused only by later work on
// the current stream, which is where the call's kernels run) and
// capture-aware (under graph capture it comes from the graph's pool), so
// the library itself holds no memory for these calls.
struct Workspace {
  at::Tensor tensor;
  Workspace(const Operands& in, std::size_t bytes) {
    if (bytes > 0)
      tensor = at::empty({static_cast<std::int64_t>(bytes)},
                         in.lead().options().dtype(at::kByte));
  }
  void* data() const { return tensor.defined() ? tensor.data_ptr() : nullptr; }
  std::size_t bytes() const { return tensor.defined() ? tensor.numel() : 0; }
};

// Runs `call(stream)` (one C ABI entry point) with the inputs' device
// current, on that device's current stream.
template <typename Call>
void launch(const Operands& in, Call&& call) {
  const c10::DeviceGuard guard(in.lead().device());
  void* stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(
                     in.lead().get_device()).stream();
  const int status = call(stream);
  TORCH_CHECK(status == 0, in.op(), " launch failed: ",
              operatorlib_status_string(status));
}

at::Tensor reduce_sum_op(const at::Tensor& input) {
  const Operands in("reduce_sum", kFloat32Only, {{&input, "input"}});
  TORCH_CHECK(input.numel() > 0, "reduce_sum: input must not be empty");
  at::Tensor out = at::empty({}, input.options());
  launch(in, [&](void* s) {
    const float* x = static_cast<const float*>(caddr(input));
    const size_t n = static_cast<size_t>(input.numel());
    const Workspace ws(in, operatorlib_reduce_sum_f32_workspace_size(x, n));
    return operatorlib_reduce_sum_f32_ws(x, static_cast<float*>(out.data_ptr()), n,
                                         ws.data(), ws.bytes(), s);
  });
  return out;
}

// softmax and rmsnorm also accept float16 (fp32 arithmetic, float16
// output): the reference binding takes float32 only
// (operatorlib_binding.cpp:60, :96) and defers FP16
// (docs/pytorch_extension.md:143-146).
at::Tensor softmax_op(const at::Tensor& input) {
  const Operands in("softmax", kFloat32OrFloat16, {{&input, "input"}});
  const auto [rows, cols] = rows_by_last(in, input, "last dimension");
  at::Tensor out = at::empty_like(input);
  launch(in, [&](void* s) {
    const Workspace ws(in, operatorlib_softmax_f32_workspace_size(rows, cols));
    return in.half()
               ? operatorlib_softmax_f16_ws(
                     static_cast<const operatorlib_half_t*>(caddr(input)),
                     static_cast<operatorlib_half_t*>(out.data_ptr()), rows, cols,
                     ws.data(), ws.bytes(), s)
               : operatorlib_softmax_f32_ws(static_cast<const float*>(caddr(input)),
                                            static_cast<float*>(out.data_ptr()), rows,
                                            cols, ws.data(), ws.bytes(), s);
  });
  return out;
}

at::Tensor transpose_op(const at::Tensor& input) {
  const Operands in("transpose", kFloat32Only, {{&input, "input"}});
  require_rank(in, input, "input", 2, "a 2D matrix");
  const int rows = extent(in.op(), "rows", input.size(0));
  const int cols = extent(in.op(), "cols", input.size(1));
  at::Tensor out = at::empty({cols, rows}, input.options());
  launch(in, [&](void* s) {
    return operatorlib_transpose_f32(static_cast<const float*>(caddr(input)),
                                     static_cast<float*>(out.data_ptr()), rows, cols, s);
  });
  return out;
}

at::Tensor rmsnorm_op(const at::Tensor& input, const at::Tensor& weight,
                      double epsilon) {
  const Operands in("rmsnorm", kFloat32OrFloat16,
                    {{&input, "input"}, {&weight, "weight"}});
  const auto [tokens, hidden] = rows_by_last(in, input, "hidden size");
  require_rank(in, weight, "weight", 1, "a 1D vector");
  TORCH_CHECK(weight.numel() == hidden, "rmsnorm: weight length ", weight.numel(),
              " does not match the hidden size ", hidden);
  TORCH_CHECK(std::isfinite(epsilon) && epsilon > 0.0,
              "rmsnorm: epsilon must be finite and > 0, got ", epsilon);
  const float eps = static_cast<float>(epsilon);
  at::Tensor out = at::empty_like(input);
  launch(in, [&](void* s) {
    const Workspace ws(in, operatorlib_rmsnorm_f32_workspace_size(tokens, hidden));
    return in.half()
               ? operatorlib_rmsnorm_f16_ws(
                     static_cast<const operatorlib_half_t*>(caddr(input)),
                     static_cast<const operatorlib_half_t*>(caddr(weight)),
                     static_cast<operatorlib_half_t*>(out.data_ptr()), tokens, hidden,
                     eps, ws.data(), ws.bytes(), s)
               : operatorlib_rmsnorm_f32_ws(static_cast<const float*>(caddr(input)),
                                            static_cast<const float*>(caddr(weight)),
                                            static_cast<float*>(out.data_ptr()), tokens,
                                            hidden, eps, ws.data(), ws.bytes(), s);
  });
  return out;
}

at::Tensor gemm_op(const at::Tensor& a, const at::Tensor& b) {
  const Operands in("gemm", kFloat32OrFloat16, {{&a, "a"}, {&b, "b"}});
  require_rank(in, a, "a", 2, "a 2D matrix");
  require_rank(in, b, "b", 2, "a 2D matrix");
  TORCH_CHECK(a.size(1) == b.size(0), "gemm: a.size(1) = ", a.size(1),
              " must equal b.size(0) = ", b.size(0));
  const int m = extent(in.op(), "M", a.size(0));
  const int k = extent(in.op(), "K", a.size(1));
  const int n = extent(in.op(), "N", b.size(1));
  at::Tensor out = at::empty({m, n}, a.options().dtype(at::kFloat));
  launch(in, [&](void* s) {
    float* c = static_cast<float*>(out.data_ptr());
    if (in.half()) {
      const auto* ha = static_cast<const operatorlib_half_t*>(caddr(a));
      const auto* hb = static_cast<const operatorlib_half_t*>(caddr(b));
      const Workspace ws(in, operatorlib_gemm_f16_workspace_size(ha, hb, m, n, k));
      return operatorlib_gemm_f16_ws(ha, hb, c, m, n, k, ws.data(), ws.bytes(), s);
    }
    const auto* fa = static_cast<const float*>(caddr(a));
    const auto* fb = static_cast<const float*>(caddr(b));
    const Workspace ws(in, operatorlib_gemm_f32_workspace_size(fa, fb, m, n, k));
    return operatorlib_gemm_f32_ws(fa, fb, c, m, n, k, ws.data(), ws.bytes(), s);
  });
  return out;
}

at::Tensor attention_op(const at::Tensor& q, const at::Tensor& k,
                        const at::Tensor& v, bool causal) {
  const Operands in("attention", kFloat32OrFloat16, {{&q, "q"}, {&k, "k"}, {&v, "v"}});
  require_rank(in, q, "q", 4, "[B,H,S,D]");
  TORCH_CHECK(k.sizes() == q.sizes() && v.sizes() == q.sizes(),
              "attention: q, k and v must have the same shape, got ", q.sizes(), ", ",
              k.sizes(), ", ", v.sizes());
  const int batch = extent(in.op(), "batch", q.size(0));
  const int heads = extent(in.op(), "heads", q.size(1));
  const int seq = extent(in.op(), "sequence", q.size(2));
  const int dim = extent(in.op(), "head dimension", q.size(3));
  TORCH_CHECK(dim <= 128, "attention: head dimension ", dim,
              " is not supported (at most 128)");
  TORCH_CHECK(static_cast<std::int64_t>(batch) * heads <= std::numeric_limits<int>::max(),
              "attention: batch * heads = ", static_cast<std::int64_t>(batch) * heads,
              " is not a positive int32");
  at::Tensor out = at::empty(q.sizes(), q.options().dtype(at::kFloat));
  launch(in, [&](void* s) {
    float* o = static_cast<float*>(out.data_ptr());
    const int c = causal ? 1 : 0;
    if (in.half()) {
      const auto* hq = static_cast<const operatorlib_half_t*>(caddr(q));
      const auto* hk = static_cast<const operatorlib_half_t*>(caddr(k));
      const auto* hv = static_cast<const operatorlib_half_t*>(caddr(v));
      const Workspace ws(in, operatorlib_attention_f16_workspace_size(hq, hk, hv, o, batch,
                                                                      heads, seq, dim, c));
      return operatorlib_attention_f16_ws(hq, hk, hv, o, batch, heads, seq, dim, c,
                                          ws.data(), ws.bytes(), s);
    }
    const auto* fq = static_cast<const float*>(caddr(q));
    const auto* fk = static_cast<const float*>(caddr(k));
    const auto* fv = static_cast<const float*>(caddr(v));
    const Workspace ws(in, operatorlib_attention_f32_workspace_size(fq, fk, fv, o, batch,
                                                                    heads, seq, dim, c));
    return operatorlib_attention_f32_ws(fq, fk, fv, o, batch, heads, seq, dim, c, ws.data(),
                                        ws.bytes(), s);
  });
  return out;
}

}  // namespace

TORCH_LIBRARY(operatorlib, m) {
  m.def("reduce_sum(Tensor input) -> Tensor");
  m.def("softmax(Tensor input) -> Tensor");
  m.def("transpose(Tensor input) -> Tensor");
  m.def("rmsnorm(Tensor input, Tensor weight, float epsilon=1e-5) -> Tensor");
  m.def("gemm(Tensor a, Tensor b) -> Tensor");
  m.def("attention(Tensor q, Tensor k, Tensor v, bool causal=False) -> Tensor");
}

TORCH_LIBRARY_IMPL(operatorlib, CUDA, m) {
  m.impl("reduce_sum", &reduce_sum_op);
  m.impl("softmax", &softmax_op);
  m.impl("transpose", &transpose_op);
  m.impl("rmsnorm", &rmsnorm_op);
  m.impl("gemm", &gemm_op);
  m.impl("attention", &attention_op);
}
