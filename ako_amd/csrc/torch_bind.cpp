// Host binding of the C ABI for PyTorch tensors (Python module _ako_torch).
//
// The HIP candidates' per-call host work -- argument checks, row views,
// output allocation from torch's caching allocator, the current stream --
// done in C++ instead of Python + ctypes. Each function makes exactly the
// checks of the corresponding Python candidate (ako_amd/ops/*_hip.py), with
// the same messages, then one call into libako_hip.so (include/ako_hip.h).
// Bad arguments raise ValueError; a failed launch raises RuntimeError.
//
// The module holds no kernels and no state: it links libako_hip.so, so tuning
// set through the C ABI applies to both bindings.

#include <torch/extension.h>
#include <ATen/hip/HIPContext.h>
#include <hip/hip_runtime.h>

#include <string>
#include <utility>

#include "ako_hip.h"

namespace py = pybind11;

namespace {

[[noreturn]] void value_error(const std::string& msg) { throw py::value_error(msg); }

// Python's repr of a torch.Size as a tuple: (), (n,), (a, b, ...).
std::string shape_str(at::IntArrayRef s) {
  if (s.empty()) return "()";
  std::string out = "(";
  for (size_t i = 0; i < s.size(); ++i) {
    if (i) out += ", ";
    out += std::to_string(s[i]);
  }
  return out + (s.size() == 1 ? ",)" : ")");
}

std::string dtype_str(at::ScalarType st) {
  switch (st) {
    case at::kFloat: return "torch.float32";
    case at::kHalf: return "torch.float16";
    case at::kBFloat16: return "torch.bfloat16";
    case at::kDouble: return "torch.float64";
    default: return std::string("torch.") + c10::toString(st);
  }
}

int dtype_code_or(at::ScalarType st) {
  switch (st) {
    case at::kFloat: return AKO_DTYPE_F32;
    case at::kHalf: return AKO_DTYPE_F16;
    case at::kBFloat16: return AKO_DTYPE_BF16;
    default: return -1;
  }
}

int dtype_code(at::ScalarType st, const char* fn) {
  const int code = dtype_code_or(st);
  if (code < 0) value_error(std::string(fn) + " supports float32/float16/bfloat16, got " + dtype_str(st));
  return code;
}

int gpu_index(const at::Tensor& t, const char* fn) {
  if (!t.is_cuda()) value_error(std::string(fn) + " requires a GPU tensor, got device " + t.device().str());
  return t.get_device();
}

bool on(const at::Tensor& t, int index) { return t.is_cuda() && t.get_device() == index; }

// A nonzero status becomes the exception type the Python candidates raise.
void check(int status, const char* fn) {
  if (status == AKO_OK) return;
  const std::string msg = std::string(fn) + ": " + ako_last_error();
  if (status == AKO_ERR_INVALID_ARGUMENT || status == AKO_ERR_UNSUPPORTED) throw py::value_error(msg);
  throw std::runtime_error(msg);
}

// Runs `launch` with device `index` current and torch's current stream of it.
template <typename F>
int on_device(int index, F&& launch) {
  int current = -1;
  if (hipGetDevice(&current) != hipSuccess) current = -1;
  if (current == index) return launch(at::hip::getCurrentHIPStream(index).stream());
  c10::DeviceGuard guard(c10::Device(c10::DeviceType::CUDA, static_cast<c10::DeviceIndex>(index)));
  return launch(at::hip::getCurrentHIPStream(index).stream());
}

// Stride between consecutive rows of the last dimension when the leading dims
// can be walked as one run of equally spaced rows, else -1. Size-1 dims are
// transparent (their stride is arbitrary and never multiplies an index); the
// innermost leading dim of size > 1 fixes the row stride, and each outer one of
// size > 1 must be that stride times the rows spanned by the dims inside it.
int64_t leading_row_stride(const at::Tensor& t) {
  const int64_t h = t.size(-1);
  int64_t row_stride = -1, spanned = 1;
  for (int64_t i = t.dim() - 2; i >= 0; --i) {
    if (t.size(i) == 1) continue;
    if (row_stride < 0) {
      row_stride = t.stride(i);
      spanned = t.size(i);
    } else if (t.stride(i) != row_stride * spanned) {
      return -1;
    } else {
      spanned *= t.size(i);
    }
  }
  if (row_stride < 0) return h;
  return row_stride >= h ? row_stride : -1;
}

// (tensor, row stride): rows of the last dimension at r * row_stride, copying
// only when the leading dims cannot be walked with one stride.
std::pair<at::Tensor, int64_t> rows_view(const at::Tensor& t) {
  if (t.is_contiguous()) return {t, t.dim() ? t.size(-1) : 1};
  if (t.dim() >= 2 && (t.stride(-1) == 1 || t.size(-1) <= 1)) {
    const int64_t row_stride = leading_row_stride(t);
    if (row_stride >= 0) return {t, row_stride};
  }
  at::Tensor c = t.contiguous();
  return {c, c.size(-1)};
}

at::Tensor empty_out(const at::Tensor& x) {
  return x.is_contiguous() ? at::empty_like(x) : at::empty(x.sizes(), x.options());
}

// Weight of a row of `hidden`: same dtype as the input or fp32 (anything else
// is widened to fp32, exactly), contiguous, on the input's device.
std::pair<at::Tensor, int> weight_arg(const at::Tensor& w, int index, int dt, int64_t hidden, const char* fn) {
  if (w.dim() != 1 || w.size(0) != hidden)
    value_error("Expected weight of shape (" + std::to_string(hidden) + ",), got " + shape_str(w.sizes()));
  if (!on(w, index)) value_error(std::string(fn) + ": weight must be on the input's device");
  at::Tensor out = w;
  int wdt = dtype_code_or(w.scalar_type());
  if (wdt != dt && wdt != AKO_DTYPE_F32) {
    out = w.to(at::kFloat);
    wdt = AKO_DTYPE_F32;
  }
  if (!out.is_contiguous()) out = out.contiguous();
  return {out, wdt};
}

// ------------------------------------------------------------------ RMSNorm --
at::Tensor rmsnorm(const at::Tensor& x, const at::Tensor& weight, double eps) {
  const char* fn = "rmsnorm_hip";
  const int index = gpu_index(x, fn);
  const int dt = dtype_code(x.scalar_type(), fn);
  const int64_t hidden = x.dim() ? x.size(-1) : 1;
  auto [w, wdt] = weight_arg(weight, index, dt, hidden, fn);
  auto [xv, sx] = rows_view(x);
  const int64_t rows = hidden ? xv.numel() / hidden : 0;
  at::Tensor y = empty_out(x);
  check(on_device(index, [&](hipStream_t s) {
          return ako_rmsnorm_fwd(xv.data_ptr(), w.data_ptr(), y.data_ptr(), rows, hidden, sx, hidden,
                                 static_cast<float>(eps), dt, wdt, s);
        }), fn);
  return y;
}

std::pair<at::Tensor, at::Tensor> rmsnorm_residual(const at::Tensor& x, const at::Tensor& residual,
                                                   const at::Tensor& weight, double eps) {
  const char* fn = "rmsnorm_residual_hip";
  const int index = gpu_index(x, fn);
  if (!x.sizes().equals(residual.sizes()))
    value_error("Shape mismatch: x " + shape_str(x.sizes()) + " vs residual " + shape_str(residual.sizes()));
  if (residual.scalar_type() != x.scalar_type() || !on(residual, index))
    value_error("rmsnorm_residual_hip: residual must match x in dtype and device");
  const int dt = dtype_code(x.scalar_type(), fn);
  const int64_t hidden = x.dim() ? x.size(-1) : 1;
  auto [w, wdt] = weight_arg(weight, index, dt, hidden, fn);
  auto [xv, sx] = rows_view(x);
  auto [rv, sr] = rows_view(residual);
  const int64_t rows = hidden ? xv.numel() / hidden : 0;
  at::Tensor y = empty_out(x);
  at::Tensor new_residual = empty_out(x);
  check(on_device(index, [&](hipStream_t s) {
          return ako_rmsnorm_residual_fwd(xv.data_ptr(), rv.data_ptr(), w.data_ptr(), y.data_ptr(),
                                          new_residual.data_ptr(), rows, hidden, sx, sr, hidden, hidden,
                                          static_cast<float>(eps), dt, wdt, s);
        }), fn);
  return {y, new_residual};
}

// --------------------------------------------------------------------- RoPE --
int style_code(const std::string& style) {
  if (style == "neox") return AKO_ROPE_NEOX;
  if (style == "interleaved") return AKO_ROPE_INTERLEAVED;
  value_error("Unknown RoPE style '" + style + "', expected one of ('neox', 'interleaved')");
}

// The reference's argument checks (ako/ops/rope_ref.py:57-70).
void validate_rope(const at::Tensor& x, const at::Tensor& cos, const at::Tensor& sin) {
  if (x.dim() != 4)
    value_error("Expected x of shape (batch, seq_len, n_heads, head_dim), got " + shape_str(x.sizes()));
  const int64_t head_dim = x.size(3);
  if (head_dim % 2 != 0) value_error("head_dim must be even, got " + std::to_string(head_dim));
  if (!cos.sizes().equals(sin.sizes()))
    value_error("cos/sin shape mismatch: " + shape_str(cos.sizes()) + " vs " + shape_str(sin.sizes()));
  if (cos.dim() != 2 || cos.size(0) != x.size(1) || cos.size(1) != head_dim / 2)
    value_error("Expected cos/sin of shape (" + std::to_string(x.size(1)) + ", " + std::to_string(head_dim / 2) +
                "), got " + shape_str(cos.sizes()));
}

at::Tensor head_view(const at::Tensor& x) { return x.stride(-1) == 1 ? x : x.contiguous(); }

at::Tensor table_arg(const at::Tensor& t, int index) {
  if (!on(t, index)) value_error("rope_hip: tables must be on the input's device, got " + t.device().str());
  at::Tensor out = dtype_code_or(t.scalar_type()) < 0 ? t.to(at::kFloat) : t;
  return out.stride(-1) == 1 ? out : out.contiguous();
}

// Both tables with one row stride (made to agree when they do not).
struct Tables {
  at::Tensor cos, sin;
  int64_t stride;
  int dtype;
};

Tables tables(const at::Tensor& cos_in, const at::Tensor& sin_in, int index) {
  at::Tensor c = table_arg(cos_in, index), s = table_arg(sin_in, index);
  if (c.stride(0) != s.stride(0) || c.scalar_type() != s.scalar_type()) {
    c = c.contiguous();
    s = s.to(c.scalar_type()).contiguous();
  }
  const int64_t st = c.size(0) > 1 ? c.stride(0) : c.size(1);
  return {c, s, st, dtype_code_or(c.scalar_type())};
}

at::Tensor rope(const at::Tensor& x, const at::Tensor& cos, const at::Tensor& sin, const std::string& style) {
  const char* fn = "rope_hip";
  const int index = gpu_index(x, fn);
  const int sc = style_code(style);
  validate_rope(x, cos, sin);
  const int dt = dtype_code(x.scalar_type(), fn);
  at::Tensor xv = head_view(x);
  Tables t = tables(cos, sin, index);
  at::Tensor y = empty_out(x);
  check(on_device(index, [&](hipStream_t s) {
          return ako_rope_fwd(xv.data_ptr(), t.cos.data_ptr(), t.sin.data_ptr(), y.data_ptr(), x.size(0),
                              x.size(1), x.size(2), x.size(3), xv.stride(0), xv.stride(1), xv.stride(2),
                              y.stride(0), y.stride(1), y.stride(2), t.stride, dt, t.dtype, sc, s);
        }), fn);
  return y;
}

std::pair<at::Tensor, at::Tensor> rope_qk(const at::Tensor& q, const at::Tensor& k, const at::Tensor& cos,
                                          const at::Tensor& sin, const std::string& style) {
  const char* fn = "rope_qk_hip";
  const int index = gpu_index(q, fn);
  const int sc = style_code(style);
  validate_rope(q, cos, sin);
  validate_rope(k, cos, sin);
  if (q.size(0) != k.size(0) || q.size(1) != k.size(1) || q.size(3) != k.size(3) ||
      q.scalar_type() != k.scalar_type() || !on(k, index))
    value_error("rope_qk_hip: q " + shape_str(q.sizes()) + " " + dtype_str(q.scalar_type()) + " and k " +
                shape_str(k.sizes()) + " " + dtype_str(k.scalar_type()) + " differ");
  const int dt = dtype_code(q.scalar_type(), fn);
  at::Tensor qv = head_view(q), kv = head_view(k);
  Tables t = tables(cos, sin, index);
  at::Tensor q_out = empty_out(q), k_out = empty_out(k);
  const int64_t st[12] = {qv.stride(0),    qv.stride(1),    qv.stride(2),    kv.stride(0),
                          kv.stride(1),    kv.stride(2),    q_out.stride(0), q_out.stride(1),
                          q_out.stride(2), k_out.stride(0), k_out.stride(1), k_out.stride(2)};
  check(on_device(index, [&](hipStream_t s) {
          return ako_rope_qk_fwd(qv.data_ptr(), kv.data_ptr(), t.cos.data_ptr(), t.sin.data_ptr(),
                                 q_out.data_ptr(), k_out.data_ptr(), q.size(0), q.size(1), q.size(2), k.size(2),
                                 q.size(3), st, st + 3, st + 6, st + 9, t.stride, dt, t.dtype, sc, s);
        }), fn);
  return {q_out, k_out};
}

at::Tensor rope_qk_cache(const at::Tensor& q, const at::Tensor& k, const c10::optional<at::Tensor>& v,
                         const at::Tensor& cos, const at::Tensor& sin, const at::Tensor& pos,
                         const at::Tensor& k_cache, const c10::optional<at::Tensor>& v_cache,
                         const std::string& style) {
  const char* fn = "rope_qk_cache_hip";
  const std::string pre = std::string(fn) + ": ";
  const int index = gpu_index(q, fn);
  const int sc = style_code(style);
  if (q.dim() != 4 || k.dim() != 4 || k_cache.dim() != 4) value_error(pre + "q, k and k_cache must be 4-D");
  const int64_t batch = q.size(0), seq = q.size(1), head_dim = q.size(3), kv_heads = k.size(2);
  if (k.size(0) != batch || k.size(1) != seq || k.size(3) != head_dim || k.scalar_type() != q.scalar_type())
    value_error(pre + "k " + shape_str(k.sizes()) + " " + dtype_str(k.scalar_type()) + " does not match q " +
                shape_str(q.sizes()) + " " + dtype_str(q.scalar_type()));
  if (k_cache.size(0) != batch || k_cache.size(1) != kv_heads || k_cache.size(3) != head_dim ||
      k_cache.scalar_type() != q.scalar_type())
    value_error(pre + "k_cache " + shape_str(k_cache.sizes()) + " " + dtype_str(k_cache.scalar_type()) +
                " is not (batch, kv_heads, cache_len, head_dim) of " + dtype_str(q.scalar_type()));
  if (v.has_value() != v_cache.has_value()) value_error(pre + "v and v_cache must both be given or both be None");
  if (v.has_value() && (!v->sizes().equals(k.sizes()) || v->scalar_type() != q.scalar_type() ||
                        !v_cache->sizes().equals(k_cache.sizes()) || v_cache->scalar_type() != q.scalar_type() ||
                        !v_cache->strides().equals(k_cache.strides())))
    value_error(pre + "v / v_cache must match k / k_cache (shapes, dtype, strides)");
  if (cos.dim() != 2 || cos.size(1) != head_dim / 2 || !sin.sizes().equals(cos.sizes()))
    value_error(pre + "tables must be (positions, " + std::to_string(head_dim / 2) + "), got " +
                shape_str(cos.sizes()));
  if (pos.scalar_type() != at::kLong || pos.numel() < 1)
    value_error(pre + "pos must be an int64 tensor holding the position");
  if (!on(k, index)) value_error(pre + "k must be on the device of q");
  if (!on(k_cache, index)) value_error(pre + "k_cache must be on the device of q");
  if (!on(pos, index)) value_error(pre + "pos must be on the device of q");
  if (v.has_value() && !on(*v, index)) value_error(pre + "v must be on the device of q");
  if (v.has_value() && !on(*v_cache, index)) value_error(pre + "v_cache must be on the device of q");
  if (k_cache.stride(3) != 1 || (v_cache.has_value() && v_cache->stride(3) != 1))
    value_error(pre + "cache rows must be contiguous in head_dim");
  const int dt = dtype_code(q.scalar_type(), fn);
  at::Tensor qv = head_view(q), kv = head_view(k);
  at::Tensor vv = v.has_value() ? head_view(*v) : at::Tensor();
  Tables t = tables(cos, sin, index);
  at::Tensor q_out = empty_out(q);
  const int64_t st[15] = {qv.stride(0), qv.stride(1), qv.stride(2), kv.stride(0), kv.stride(1), kv.stride(2),
                          vv.defined() ? vv.stride(0) : 0, vv.defined() ? vv.stride(1) : 0,
                          vv.defined() ? vv.stride(2) : 0, q_out.stride(0), q_out.stride(1), q_out.stride(2),
                          k_cache.stride(0), k_cache.stride(2), k_cache.stride(1)};
  check(on_device(index, [&](hipStream_t s) {
          return ako_rope_qk_cache_fwd(qv.data_ptr(), kv.data_ptr(), vv.defined() ? vv.data_ptr() : nullptr,
                                       t.cos.data_ptr(), t.sin.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(),
                                       v_cache.has_value() ? v_cache->data_ptr() : nullptr,
                                       static_cast<const int64_t*>(pos.data_ptr()), batch, seq, q.size(2), kv_heads,
                                       head_dim, st, st + 3, st + 6, st + 9, st + 12, k_cache.size(2),
                                       t.cos.size(0), t.stride, dt, t.dtype, sc, s);
        }), fn);
  return q_out;
}

// ------------------------------------------------------------------- SwiGLU --
at::Tensor swiglu(const at::Tensor& gate, const at::Tensor& up) {
  const char* fn = "swiglu_hip";
  const int index = gpu_index(gate, fn);
  if (!gate.sizes().equals(up.sizes()))
    value_error("Shape mismatch: gate " + shape_str(gate.sizes()) + " vs up " + shape_str(up.sizes()));
  if (up.scalar_type() != gate.scalar_type() || !on(up, index))
    value_error("swiglu_hip: up must match gate in dtype and device");
  const int dt = dtype_code(gate.scalar_type(), fn);
  const int64_t n = gate.dim() ? gate.size(-1) : 1;
  auto [gv, sg] = rows_view(gate);
  auto [uv, su] = rows_view(up);
  const int64_t rows = n ? gv.numel() / n : 0;
  at::Tensor y = empty_out(gate);
  check(on_device(index, [&](hipStream_t s) {
          return ako_swiglu_fwd(gv.data_ptr(), uv.data_ptr(), y.data_ptr(), rows, n, sg, su, n, dt, s);
        }), fn);
  return y;
}

// The stream this binding launches on, for tests: torch's current stream.
int64_t current_stream(int64_t index) {
  return reinterpret_cast<int64_t>(at::hip::getCurrentHIPStream(static_cast<c10::DeviceIndex>(index)).stream());
}

// The row walk rows_view takes for t, for host tests: (copied, row stride).
std::pair<bool, int64_t> row_walk(const at::Tensor& t) {
  auto [v, stride] = rows_view(t);
  return {!v.is_same(t), stride};
}

}  // namespace

PYBIND11_MODULE(_ako_torch, m) {
  m.doc() = "PyTorch binding of libako_hip.so's C ABI (the HIP candidates' host path)";
  m.def("abi_version", [] { return ako_abi_version(); });
  m.def("rmsnorm", &rmsnorm, py::arg("x"), py::arg("weight"), py::arg("eps") = 1e-6);
  m.def("rmsnorm_residual", &rmsnorm_residual, py::arg("x"), py::arg("residual"), py::arg("weight"),
        py::arg("eps") = 1e-6);
  m.def("rope", &rope, py::arg("x"), py::arg("cos"), py::arg("sin"), py::arg("style") = "neox");
  m.def("rope_qk", &rope_qk, py::arg("q"), py::arg("k"), py::arg("cos"), py::arg("sin"),
        py::arg("style") = "neox");
  m.def("rope_qk_cache", &rope_qk_cache, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("cos"),
        py::arg("sin"), py::arg("pos"), py::arg("k_cache"), py::arg("v_cache"), py::arg("style") = "neox");
  m.def("swiglu", &swiglu, py::arg("gate"), py::arg("up"));
  m.def("current_stream", &current_stream);
  m.def("row_walk", &row_walk, py::arg("t"));
}
