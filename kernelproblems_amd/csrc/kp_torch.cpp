// Native tensor-level wrappers of the entry points of kernelproblems_amd.fused
// (RMSNorm, embedding, RoPE, FSDP unshard, SwiGLU, cross-entropy).  Each checks
// the tensors, finds the row layout, allocates outputs and workspace with
// torch's caching allocator, and calls the C ABI (include/kp.h) on the
// device's current stream, in one native call, so that a drop-in's host time
// per call is the kernel launches plus a few allocations rather than Python
// argument marshalling (a small fragment's kernel runs for less time than
// that marshalling took).  The index-checking flag is the caller's: fused.py
// owns the per-device flag and raises after the call when checking is on.
//
// Built with g++ against torch's headers (no device code here) into the
// Python module _kp_torch, linked to libkp_hip.so.  Errors: a bad tensor raises
// RuntimeError with the same text as the Python checks; a non-zero status from
// the C ABI raises kernelproblems_amd._lib.KPError with the library's message.
#include <torch/extension.h>

#include <ATen/TensorUtils.h>
#include <c10/hip/HIPStream.h>

#include <cmath>
#include <optional>
#include <string>
#include <vector>

#include "kp.h"

namespace py = pybind11;
using at::Tensor;

namespace {

std::string dtype_name(at::ScalarType t) {
  switch (t) {
    case at::kBFloat16: return "torch.bfloat16";
    case at::kFloat: return "torch.float32";
    case at::kHalf: return "torch.float16";
    case at::kDouble: return "torch.float64";
    case at::kComplexFloat: return "torch.complex64";
    case at::kLong: return "torch.int64";
    case at::kInt: return "torch.int32";
    default: return std::string("torch.") + c10::toString(t);
  }
}

std::string shape_str(at::IntArrayRef s) {
  std::string r = "(";
  for (size_t i = 0; i < s.size(); ++i) r += std::to_string(s[i]) + (s.size() == 1 ? "," : (i + 1 < s.size() ? ", " : ""));
  return r + ")";
}

[[noreturn]] void fail(const std::string& msg) { throw std::runtime_error(msg); }

// A non-zero status of a C-ABI call: raise the package's KPError.
void check(const char* fn, int st) {
  if (st == KP_OK) return;
  py::object cls = py::module_::import("kernelproblems_amd._lib").attr("KPError");
  const char* m = kp_last_error_message();
  py::object msg = py::bytes(m ? m : "").attr("decode")("utf-8", "replace");
  py::object err = cls(fn, st, msg);
  PyErr_SetObject(cls.ptr(), err.ptr());
  throw py::error_already_set();
}

void need_gpu(const std::string& name, const Tensor& t, std::optional<at::ScalarType> dt = at::kBFloat16) {
  if (!t.is_cuda())
    fail(name + ": expected a GPU tensor, got device " + t.device().str() + " (no CPU path exists)");
  if (dt && t.scalar_type() != *dt)
    fail(name + ": expected dtype " + dtype_name(*dt) + ", got " + dtype_name(t.scalar_type()));
}

// The tensor's device made current (HIP launches on the current device) and
// that device's current stream.  Passed as a temporary in a C call's argument
// list, so the device stays current until the call returns.
struct DeviceStream {
  c10::DeviceGuard guard;
  void* stream;
  explicit DeviceStream(const Tensor& t)
      : guard(t.device()), stream(c10::hip::getCurrentHIPStream(t.device().index()).stream()) {}
  operator void*() const { return stream; }
};
DeviceStream stream_of(const Tensor& t) { return DeviceStream(t); }

void* ptr(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

// The caller's per-device out-of-range flag (int32), if any.
int32_t* flag_ptr(const std::optional<Tensor>& flag) {
  return flag ? static_cast<int32_t*>(flag->data_ptr()) : nullptr;
}

// t viewed as [m, n] rows with unit inner stride: (tensor, row stride, m);
// copies to contiguous only when no such view exists.
struct Rows {
  Tensor t;
  int64_t stride;
  int64_t m;
};
Rows as_rows(Tensor t, int64_t n) {
  const int64_t numel = t.numel();
  if (n <= 0 || numel % n != 0)
    fail("tensor of " + std::to_string(numel) + " elements is not a whole number of rows of " + std::to_string(n));
  const int64_t m = numel / n;
  if (m == 0) return {t, n, 0};
  if (t.is_contiguous()) return {t, n, m};
  const std::vector<int64_t> shape{m, n};
  const auto st = at::detail::computeStride(t.sizes(), t.strides(), shape);
  if (st && (n == 1 || (*st)[1] == 1)) return {t, (*st)[0], m};
  t = t.contiguous();
  return {t, n, m};
}

// Element i of the flattened weight sits at (i / seg_len) * seg_stride +
// i % seg_len: contiguous vectors and 2-D row-strided views (an [8, 512]
// slice of an FSDP flat buffer).
struct Segments {
  Tensor w;
  int64_t len, stride;
};
Segments weight_segments(Tensor w, int64_t n) {
  if (w.numel() != n) fail("weight has " + std::to_string(w.numel()) + " elements, expected " + std::to_string(n));
  if (w.dim() == 1 && (w.stride(0) == 1 || n == 1)) return {w, n, n};
  if (w.dim() == 2 && (w.stride(1) == 1 || w.size(1) == 1)) return {w, w.size(1), w.stride(0)};
  if (!w.is_contiguous()) w = w.contiguous();
  return {w, n, n};
}

py::object opt(const Tensor& t) { return t.defined() ? py::cast(t) : py::none(); }

// ------------------------------------------------------------------ RMSNorm
py::tuple rms_norm(const std::vector<Tensor>& x_terms, const std::optional<Tensor>& weight, double eps, int64_t n,
                   bool return_h, bool return_rstd) {
  if (x_terms.empty() || x_terms.size() > 3) fail("rms_norm: 1..3 input terms");
  const Tensor& x0 = x_terms[0];
  need_gpu("rms_norm input", x0);
  const auto dev = x0.device();
  Tensor rows[3];
  const void* ptrs[3];
  int64_t strides[3];
  int64_t m = 0;
  for (size_t i = 0; i < x_terms.size(); ++i) {
    const Tensor& t = x_terms[i];
    need_gpu("rms_norm input " + std::to_string(i), t);
    if (t.numel() != x0.numel() || t.device() != dev)
      fail("rms_norm: input terms must have the same number of elements and device");
    Rows r = as_rows(t, n);
    rows[i] = r.t;
    ptrs[i] = r.t.data_ptr();
    strides[i] = r.stride;
    m = r.m;
  }
  Segments ws{Tensor(), n, n};
  if (weight) {
    need_gpu("rms_norm weight", *weight);
    ws = weight_segments(*weight, n);
  }
  const auto bf = x0.options().dtype(at::kBFloat16);
  Tensor y = at::empty(x0.sizes(), bf);
  Tensor h = (return_h && x_terms.size() > 1) ? at::empty(x0.sizes(), bf) : Tensor();
  Tensor rstd = return_rstd ? at::empty({m}, bf.dtype(at::kFloat)) : Tensor();
  check("kp_rmsnorm_fwd_bf16",
        kp_rmsnorm_fwd_bf16(ptrs, strides, (int)x_terms.size(), ptr(ws.w), ws.len, ws.stride, ptr(h), n, y.data_ptr(),
                            n, static_cast<float*>(ptr(rstd)), m, n, (float)eps, stream_of(x0)));
  py::object ho = h.defined() ? py::cast(h) : (return_h ? py::cast(x0) : py::none());
  return py::make_tuple(ho, y, opt(rstd));
}

// The backward's operands as rows: dy terms, x terms, weight segments and the
// residual (the checks and layout rules of rms_norm).
struct BwdOperands {
  Tensor dyr[3], xr[3], res;
  const void* dyp[3];
  const void* xp[3];
  int64_t dys[3], xs[3];
  int n_dy = 0, n_x = 0;
  int64_t m = 0, res_s = 0;
  Segments ws;
};
void bwd_operands(const std::string& who, const std::vector<Tensor>& dy_terms, const std::vector<Tensor>& x_terms,
                  const std::optional<Tensor>& weight, int64_t n, const std::optional<Tensor>& dx_residual,
                  BwdOperands& o) {
  if (dy_terms.empty() || dy_terms.size() > 3 || x_terms.empty() || x_terms.size() > 3)
    fail(who + ": 1..3 grad terms and 1..3 input terms");
  const Tensor& dy0 = dy_terms[0];
  need_gpu(who + " grad_out", dy0);
  for (size_t i = 0; i < dy_terms.size(); ++i) {
    const Tensor& t = dy_terms[i];
    need_gpu(who + " grad term " + std::to_string(i), t);
    if (t.numel() != dy0.numel()) fail(who + ": grad terms must have the same number of elements");
    Rows r = as_rows(t, n);
    o.dyr[i] = r.t;
    o.dyp[i] = r.t.data_ptr();
    o.dys[i] = r.stride;
    o.m = r.m;
  }
  for (size_t i = 0; i < x_terms.size(); ++i) {
    const Tensor& t = x_terms[i];
    need_gpu(who + " input term " + std::to_string(i), t);
    if (t.numel() != dy0.numel()) fail(who + ": input and grad must have the same number of elements");
    Rows r = as_rows(t, n);
    o.xr[i] = r.t;
    o.xp[i] = r.t.data_ptr();
    o.xs[i] = r.stride;
  }
  o.n_dy = (int)dy_terms.size();
  o.n_x = (int)x_terms.size();
  o.ws = Segments{Tensor(), n, n};
  if (weight) {
    need_gpu(who + " weight", *weight);
    o.ws = weight_segments(*weight, n);
  }
  o.res_s = n;
  if (dx_residual) {
    need_gpu(who + " residual", *dx_residual);
    Rows r = as_rows(*dx_residual, n);
    o.res = r.t;
    o.res_s = r.stride;
  }
}

// Weight-gradient outputs for dw mode "f32", "f32_bf16", "bf16" or none.
void dw_outputs(const std::string& who, const std::optional<std::string>& dw, bool have_weight, int64_t n,
                const at::TensorOptions& bf, Tensor& dw_f32, Tensor& dw_bf16) {
  if (!dw) return;
  if (!have_weight) fail(who + ": no weight, no weight gradient");
  if (*dw == "f32" || *dw == "f32_bf16") dw_f32 = at::empty({n}, bf.dtype(at::kFloat));
  else if (*dw == "bf16") dw_bf16 = at::empty({n}, bf);
  else throw py::value_error(who + ": unknown dw mode '" + *dw + "'");
}

Tensor dw_view(const Tensor& dw_f32, const Tensor& dw_bf16, const std::optional<Tensor>& weight) {
  Tensor out = dw_f32.defined() ? dw_f32 : dw_bf16;
  if (weight && out.defined()) out = out.view(weight->sizes());
  return out;
}

py::tuple rms_norm_backward(const std::vector<Tensor>& dy_terms, const std::vector<Tensor>& x_terms,
                            const std::optional<Tensor>& rstd, const std::optional<Tensor>& weight, double eps,
                            int64_t n, const std::optional<Tensor>& dx_residual, bool want_dx,
                            const std::optional<std::string>& dw) {
  const std::string who = "rms_norm_backward";
  BwdOperands o;
  bwd_operands(who, dy_terms, x_terms, weight, n, dx_residual, o);
  Tensor rstd_t;
  if (rstd) {
    need_gpu(who + " rstd", *rstd, at::kFloat);
    if (rstd->numel() != o.m)
      fail(who + ": rstd has " + std::to_string(rstd->numel()) + " values, expected " + std::to_string(o.m));
    rstd_t = rstd->contiguous();
  }
  const Tensor& dy0 = dy_terms[0];
  const auto bf = dy0.options().dtype(at::kBFloat16);
  Tensor dx = at::empty(x_terms[0].sizes(), bf);
  Tensor dw_f32, dw_bf16;
  dw_outputs(who, dw, weight.has_value(), n, bf, dw_f32, dw_bf16);
  size_t ws_bytes = 0;
  Tensor wsp;
  if (dw) {
    ws_bytes = kp_rmsnorm_bwd_workspace_size(o.m, n);
    wsp = at::empty({(int64_t)std::max<size_t>(ws_bytes, 16)}, bf.dtype(at::kByte));
  }
  check("kp_rmsnorm_bwd_bf16",
        kp_rmsnorm_bwd_bf16(o.dyp, o.dys, o.n_dy, o.xp, o.xs, o.n_x, static_cast<const float*>(ptr(rstd_t)),
                            ptr(o.ws.w), o.ws.len, o.ws.stride, ptr(o.res), o.res_s, dx.data_ptr(), n,
                            static_cast<float*>(ptr(dw_f32)), ptr(dw_bf16), (dw && *dw == "f32_bf16") ? 1 : 0, o.m,
                            n, (float)eps, ptr(wsp), ws_bytes, stream_of(dy0)));
  return py::make_tuple(want_dx ? py::cast(dx) : py::none(), opt(dw_view(dw_f32, dw_bf16, weight)));
}

py::tuple rms_norm_forward_backward(const std::vector<Tensor>& dy_terms, const std::vector<Tensor>& x_terms,
                                    const std::optional<Tensor>& weight, double eps, int64_t n,
                                    const std::optional<Tensor>& dx_residual, const std::optional<std::string>& dw,
                                    bool return_h, bool return_rstd) {
  const std::string who = "rms_norm_forward_backward";
  BwdOperands o;
  bwd_operands(who, dy_terms, x_terms, weight, n, dx_residual, o);
  const Tensor& dy0 = dy_terms[0];
  const auto bf = dy0.options().dtype(at::kBFloat16);
  const auto shape = x_terms[0].sizes();
  Tensor y = at::empty(shape, bf);
  Tensor dx = at::empty(shape, bf);
  Tensor h = (return_h && x_terms.size() > 1) ? at::empty(shape, bf) : Tensor();
  Tensor rstd = return_rstd ? at::empty({o.m}, bf.dtype(at::kFloat)) : Tensor();
  Tensor dw_f32, dw_bf16;
  dw_outputs(who, dw, weight.has_value(), n, bf, dw_f32, dw_bf16);
  const size_t ws_bytes = kp_rmsnorm_fwd_bwd_workspace_size(o.m, n);
  Tensor wsp = at::empty({(int64_t)std::max<size_t>(ws_bytes, 16)}, bf.dtype(at::kByte));
  check("kp_rmsnorm_fwd_bwd_bf16",
        kp_rmsnorm_fwd_bwd_bf16(o.dyp, o.dys, o.n_dy, o.xp, o.xs, o.n_x, ptr(o.ws.w), o.ws.len, o.ws.stride, ptr(h),
                                n, y.data_ptr(), n, static_cast<float*>(ptr(rstd)), ptr(o.res), o.res_s,
                                dx.data_ptr(), n, static_cast<float*>(ptr(dw_f32)), ptr(dw_bf16),
                                (dw && *dw == "f32_bf16") ? 1 : 0, o.m, n, (float)eps, wsp.data_ptr(), ws_bytes,
                                stream_of(dy0)));
  py::object ho = h.defined() ? py::cast(h) : (return_h ? py::cast(x_terms[0]) : py::none());
  return py::make_tuple(y, dx, opt(dw_view(dw_f32, dw_bf16, weight)), ho, opt(rstd));
}

// ---------------------------------------------------------------- embedding
void index_info(const Tensor& indices, Tensor& idx, int& ib) {
  if (!indices.is_cuda()) fail("indices must be a GPU tensor, got " + indices.device().str());
  if (indices.scalar_type() != at::kLong && indices.scalar_type() != at::kInt)
    fail("indices must be int64 or int32, got " + dtype_name(indices.scalar_type()));
  idx = indices.contiguous();
  ib = (int)idx.element_size();
}

Tensor embedding(const Tensor& table, const Tensor& indices, const std::optional<Tensor>& flag) {
  need_gpu("embedding weight", table);
  if (table.dim() != 2) fail("embedding: weight must be 2-D");
  Tensor idx;
  int ib = 0;
  index_info(indices, idx, ib);
  const int64_t V = table.size(0), D = table.size(1);
  Rows t = as_rows(table, D);
  std::vector<int64_t> shape(indices.sizes().begin(), indices.sizes().end());
  shape.push_back(D);
  Tensor out = at::empty(shape, table.options().dtype(at::kBFloat16));
  check("kp_embedding_fwd_bf16",
        kp_embedding_fwd_bf16(t.t.data_ptr(), V, D, t.stride, idx.data_ptr(), ib, idx.numel(), out.data_ptr(), D,
                              flag_ptr(flag), stream_of(table)));
  return out;
}

py::tuple embedding_rms_norm(const Tensor& table, const Tensor& indices, const std::optional<Tensor>& weight,
                             double eps, bool return_h, bool return_rstd, const std::optional<Tensor>& flag) {
  need_gpu("embedding_rms_norm table", table);
  if (table.dim() != 2) fail("embedding_rms_norm: table must be 2-D");
  Tensor idx;
  int ib = 0;
  index_info(indices, idx, ib);
  const int64_t V = table.size(0), D = table.size(1);
  Rows t = as_rows(table, D);
  const int64_t T = idx.numel();
  std::vector<int64_t> shape(indices.sizes().begin(), indices.sizes().end());
  shape.push_back(D);
  const auto bf = table.options().dtype(at::kBFloat16);
  Tensor y = at::empty(shape, bf);
  Tensor h = return_h ? at::empty(shape, bf) : Tensor();
  Tensor rstd = return_rstd ? at::empty(indices.sizes(), bf.dtype(at::kFloat)) : Tensor();
  Segments ws{Tensor(), D, D};
  if (weight) {
    need_gpu("embedding_rms_norm weight", *weight);
    ws = weight_segments(*weight, D);
  }
  const int st = kp_embedding_rmsnorm_fwd_bf16(t.t.data_ptr(), V, t.stride, idx.data_ptr(), ib, T, ptr(ws.w), ws.len,
                                               ws.stride, ptr(h), D, y.data_ptr(), D, static_cast<float*>(ptr(rstd)), D,
                                               (float)eps, flag_ptr(flag),
                                               stream_of(table));
  if (st == KP_EUNSUPPORTED) {  // no fused kernel for this row shape: the gather, then the norm
    Tensor emb = embedding(table, indices, flag);
    py::tuple r = rms_norm({emb}, weight, eps, D, false, return_rstd);
    py::object rs = return_rstd ? py::cast(r[2].cast<Tensor>().view(indices.sizes())) : py::none();
    return py::make_tuple(return_h ? py::cast(emb) : py::none(), r[1], rs);
  }
  check("kp_embedding_rmsnorm_fwd_bf16", st);
  return py::make_tuple(opt(h), y, opt(rstd));
}

Tensor embedding_dense_backward(const Tensor& grad_output, const Tensor& indices, int64_t num_weights,
                                int64_t padding_idx, bool scale_grad_by_freq, bool out_f32, bool round_to_bf16,
                                const std::optional<Tensor>& flag) {
  need_gpu("embedding_dense_backward grad_output", grad_output);
  Tensor idx;
  int ib = 0;
  index_info(indices, idx, ib);
  const int64_t T = idx.numel();
  const int64_t D = grad_output.dim() ? grad_output.size(-1) : 1;
  if (grad_output.numel() != T * D)
    fail("embedding_dense_backward: grad_output " + shape_str(grad_output.sizes()) + " does not match " +
         std::to_string(T) + " indices");
  Rows g = as_rows(grad_output, D);
  Tensor out = at::empty({num_weights, D}, grad_output.options().dtype(out_f32 ? at::kFloat : at::kBFloat16));
  const size_t ws_bytes = kp_embedding_bwd_workspace_size(T, num_weights, D);
  Tensor wsp = at::empty({(int64_t)std::max<size_t>(ws_bytes, 16)}, grad_output.options().dtype(at::kByte));
  check("kp_embedding_bwd_bf16",
        kp_embedding_bwd_bf16(g.t.data_ptr(), g.stride, idx.data_ptr(), ib, T, num_weights, D, padding_idx,
                              scale_grad_by_freq ? 1 : 0, out.data_ptr(), out_f32 ? KP_DTYPE_F32 : KP_DTYPE_BF16,
                              round_to_bf16 ? 1 : 0, wsp.data_ptr(), ws_bytes,
                              flag_ptr(flag), stream_of(grad_output)));
  return out;
}

// The RMSNorm backward (with its forward when rstd is None) whose residual
// output g = dx_residual + dx feeds the dense embedding backward of the same
// tokens: one row pass that sums g straight into the table
// (kp_rmsnorm_embedding_bwd_bf16).  Layouts without a fused kernel run the
// norm entry point and then the embedding backward of its stored g (same y,
// g and table bits; the weight gradient groups its rows differently).
// Returns (y or None, dw or None, table).
py::tuple rms_norm_embedding_backward(const std::vector<Tensor>& dy_terms, const Tensor& x,
                                      const std::optional<Tensor>& rstd, const std::optional<Tensor>& weight,
                                      double eps, int64_t n, const Tensor& dx_residual, bool want_y,
                                      const std::optional<std::string>& dw, const Tensor& indices,
                                      int64_t num_weights, int64_t padding_idx, bool out_f32, bool round_to_bf16,
                                      const std::optional<Tensor>& flag) {
  const std::string who = "rms_norm_embedding_backward";
  BwdOperands o;
  bwd_operands(who, dy_terms, {x}, weight, n, dx_residual, o);
  if (rstd && want_y) fail(who + ": y is the forward's output: pass rstd=None to compute it");
  Tensor rstd_t;
  if (rstd) {
    need_gpu(who + " rstd", *rstd, at::kFloat);
    if (rstd->numel() != o.m)
      fail(who + ": rstd has " + std::to_string(rstd->numel()) + " values, expected " + std::to_string(o.m));
    rstd_t = rstd->contiguous();
  }
  Tensor idx;
  int ib = 0;
  index_info(indices, idx, ib);
  if (idx.numel() != o.m)
    fail(who + ": " + std::to_string(idx.numel()) + " indices for " + std::to_string(o.m) + " rows");
  const Tensor& dy0 = dy_terms[0];
  const auto bf = dy0.options().dtype(at::kBFloat16);
  Tensor y = want_y ? at::empty(x.sizes(), bf) : Tensor();
  Tensor dw_f32, dw_bf16;
  dw_outputs(who, dw, weight.has_value(), n, bf, dw_f32, dw_bf16);
  Tensor table = at::empty({num_weights, n}, dy0.options().dtype(out_f32 ? at::kFloat : at::kBFloat16));
  const size_t ws_bytes = kp_rmsnorm_embedding_bwd_workspace_size(o.m, n, num_weights);
  Tensor wsp = at::empty({(int64_t)std::max<size_t>(ws_bytes, 16)}, bf.dtype(at::kByte));
  const int st = kp_rmsnorm_embedding_bwd_bf16(
      o.dyp, o.dys, o.n_dy, o.xp[0], o.xs[0], static_cast<const float*>(ptr(rstd_t)), ptr(o.ws.w), o.ws.len,
      o.ws.stride, ptr(o.res), o.res_s, ptr(y), n, nullptr, static_cast<float*>(ptr(dw_f32)), ptr(dw_bf16),
      (dw && *dw == "f32_bf16") ? 1 : 0, o.m, n, (float)eps, idx.data_ptr(), ib, num_weights, padding_idx,
      table.data_ptr(), out_f32 ? KP_DTYPE_F32 : KP_DTYPE_BF16, round_to_bf16 ? 1 : 0, wsp.data_ptr(), ws_bytes,
      flag_ptr(flag), stream_of(dy0));
  if (st == KP_EUNSUPPORTED) {  // no fused row pass for this layout: the norm, then the embedding backward of g
    wsp = Tensor();
    Tensor g;
    py::object dwo;
    if (rstd) {
      py::tuple r = rms_norm_backward(dy_terms, {x}, rstd, weight, eps, n, dx_residual, true, dw);
      g = r[0].cast<Tensor>();
      dwo = r[1];
    } else {
      py::tuple r = rms_norm_forward_backward(dy_terms, {x}, weight, eps, n, dx_residual, dw, false, false);
      if (want_y) y = r[0].cast<Tensor>();
      g = r[1].cast<Tensor>();
      dwo = r[2];
    }
    Tensor t = embedding_dense_backward(g, indices, num_weights, padding_idx, false, out_f32, round_to_bf16, flag);
    return py::make_tuple(opt(y), dwo, t);
  }
  check("kp_rmsnorm_embedding_bwd_bf16", st);
  return py::make_tuple(opt(y), opt(dw_view(dw_f32, dw_bf16, weight)), table);
}

// ------------------------------------------------------------- FSDP unshard
std::vector<Tensor> unshard(Tensor flat, int64_t shards, const std::vector<int64_t>& split_sizes,
                            const std::vector<int64_t>& keep) {
  need_gpu("unshard buffer", flat);
  int64_t row_len = 0, stride = 0;
  if (flat.dim() == 1) {
    if (shards <= 0 || flat.numel() % shards != 0)
      fail("unshard: " + std::to_string(flat.numel()) + " elements do not split into " + std::to_string(shards) +
           " shards");
    row_len = flat.numel() / shards;
    if (flat.stride(0) != 1 && flat.numel() > 1) flat = flat.contiguous();
    stride = row_len;
  } else if (flat.dim() == 2 && flat.size(0) == shards && (flat.stride(1) == 1 || flat.size(1) == 1)) {
    row_len = flat.size(1);
    stride = flat.stride(0);
  } else {
    fail("unshard: expected a 1-D buffer or a [" + std::to_string(shards) + ", L] view, got " +
         shape_str(flat.sizes()));
  }
  int64_t total = 0;
  for (int64_t v : split_sizes) total += v;
  if (total != row_len)
    fail("unshard: split sizes sum to " + std::to_string(total) + ", shard row has " + std::to_string(row_len));
  std::vector<int64_t> offs{0};
  for (int64_t v : split_sizes) offs.push_back(offs.back() + v);
  const int64_t nseg = (int64_t)split_sizes.size();
  std::vector<Tensor> outs;
  for (int64_t i : keep) {
    if (i < 0 || i >= nseg) throw py::index_error("unshard: segment index " + std::to_string(i) + " out of range");
    outs.push_back(at::empty({shards, split_sizes[i]}, flat.options().dtype(at::kBFloat16)));
  }
  for (size_t start = 0; start < outs.size(); start += 16) {
    const size_t cnt = std::min<size_t>(16, outs.size() - start);
    int64_t off[16], len[16];
    void* dst[16];
    for (size_t j = 0; j < cnt; ++j) {
      off[j] = offs[keep[start + j]];
      len[j] = split_sizes[keep[start + j]];
      dst[j] = outs[start + j].data_ptr();
    }
    check("kp_unshard_bf16", kp_unshard_bf16(flat.data_ptr(), shards, stride, off, len, dst, (int)cnt, stream_of(flat)));
  }
  return outs;
}

// ------------------------------------------------------------ SwiGLU gate
// Same-shape bf16 GPU operands as [rows, N] with unit inner stride.
std::vector<Rows> same_rows(const std::string& name, const std::vector<Tensor>& ts, int64_t& n) {
  const Tensor& t0 = ts[0];
  for (size_t i = 0; i < ts.size(); ++i) {
    const Tensor& t = ts[i];
    need_gpu(name + " operand " + std::to_string(i), t);
    if (t.numel() != t0.numel() || (t.dim() && (t0.dim() == 0 || t.size(-1) != t0.size(-1))))
      fail(name + ": operand " + std::to_string(i) + " has shape " + shape_str(t.sizes()) + ", expected " +
           shape_str(t0.sizes()));
    if (t.device() != t0.device()) fail(name + ": operands on different devices");
  }
  n = t0.dim() ? t0.size(-1) : 1;
  std::vector<Rows> rows;
  for (const Tensor& t : ts) rows.push_back((n == 0 || t0.numel() == 0) ? Rows{t, std::max<int64_t>(n, 1), 0}
                                                                         : as_rows(t, n));
  return rows;
}

Tensor swiglu(const Tensor& a, const Tensor& b) {
  int64_t n = 0;
  auto r = same_rows("swiglu", {a, b}, n);
  Tensor out = at::empty(a.sizes(), a.options().dtype(at::kBFloat16));
  if (r[0].m)
    check("kp_swiglu_fwd_bf16", kp_swiglu_fwd_bf16(r[0].t.data_ptr(), r[0].stride, r[1].t.data_ptr(), r[1].stride,
                                                   out.data_ptr(), n, r[0].m, n, stream_of(a)));
  return out;
}

py::tuple swiglu_backward(const Tensor& g, const Tensor& s, const Tensor& b, const Tensor& a) {
  int64_t n = 0;
  auto r = same_rows("swiglu_backward", {g, s, b, a}, n);
  const auto bf = g.options().dtype(at::kBFloat16);
  Tensor db = at::empty(g.sizes(), bf), da = at::empty(g.sizes(), bf);
  if (r[0].m)
    check("kp_swiglu_bwd_bf16",
          kp_swiglu_bwd_bf16(r[0].t.data_ptr(), r[0].stride, r[1].t.data_ptr(), r[1].stride, r[2].t.data_ptr(),
                             r[2].stride, r[3].t.data_ptr(), r[3].stride, db.data_ptr(), n, da.data_ptr(), n, r[0].m,
                             n, stream_of(g)));
  return py::make_tuple(db, da);
}

Tensor silu(const Tensor& a) {
  int64_t n = 0;
  auto r = same_rows("silu", {a}, n);
  Tensor out = at::empty(a.sizes(), a.options().dtype(at::kBFloat16));
  if (r[0].m)
    check("kp_silu_bf16", kp_silu_bf16(r[0].t.data_ptr(), r[0].stride, out.data_ptr(), n, r[0].m, n, stream_of(a)));
  return out;
}

py::tuple swiglu_forward_backward(const Tensor& a, const Tensor& b, const Tensor& g) {
  int64_t n = 0;
  auto r = same_rows("swiglu_forward_backward", {a, b, g}, n);
  const auto bf = a.options().dtype(at::kBFloat16);
  Tensor h = at::empty(a.sizes(), bf), db = at::empty(a.sizes(), bf), da = at::empty(a.sizes(), bf);
  if (r[0].m)
    check("kp_swiglu_fwd_bwd_bf16",
          kp_swiglu_fwd_bwd_bf16(r[0].t.data_ptr(), r[0].stride, r[1].t.data_ptr(), r[1].stride, r[2].t.data_ptr(),
                                 r[2].stride, h.data_ptr(), n, db.data_ptr(), n, da.data_ptr(), n, r[0].m, n,
                                 stream_of(a)));
  return py::make_tuple(h, db, da);
}

// ------------------------------------------------------------ cross-entropy
// Targets as a flat unit-stride int tensor of M entries on the logits' device.
Tensor targets_of(const py::object& targets, int64_t M, const at::Device& dev, int& tb) {
  if (!THPVariable_Check(targets.ptr())) fail("cross_entropy: targets must be a tensor on the logits' device");
  Tensor t = targets.cast<Tensor>();
  if (t.device() != dev) fail("cross_entropy: targets must be a tensor on the logits' device");
  if (t.scalar_type() != at::kLong && t.scalar_type() != at::kInt)
    fail("cross_entropy: targets must be int64 or int32, got " + dtype_name(t.scalar_type()));
  if (t.numel() != M) fail("cross_entropy: " + std::to_string(t.numel()) + " targets for " + std::to_string(M) + " rows");
  t = t.reshape({-1});
  if (M > 1 && t.stride(0) != 1) t = t.contiguous();
  tb = (int)t.element_size();
  return t;
}

py::tuple cross_entropy_loss(const Tensor& logits, const py::object& targets, int64_t ignore_index, double scale,
                             bool return_lse, const std::optional<Tensor>& flag) {
  need_gpu("cross_entropy logits", logits);
  const auto dev = logits.device();
  const int64_t V = logits.dim() ? logits.size(-1) : 1;
  Rows l = as_rows(logits, V);
  int tb = 0;
  Tensor t = targets_of(targets, l.m, dev, tb);
  const auto f32 = logits.options().dtype(at::kFloat);
  Tensor loss = at::empty({}, f32), tw = at::empty({}, f32);
  Tensor lse;
  if (return_lse) {
    auto sz = logits.sizes();
    lse = at::empty(std::vector<int64_t>(sz.begin(), sz.end() - (sz.empty() ? 0 : 1)), f32);
  }
  const size_t ws_bytes = kp_cross_entropy_fwd_workspace_size(l.m);
  Tensor wsp = at::empty({(int64_t)std::max<size_t>(ws_bytes, 8)}, logits.options().dtype(at::kByte));
  check("kp_cross_entropy_fwd_bf16",
        kp_cross_entropy_fwd_bf16(l.t.data_ptr(), l.stride, l.m, V, t.data_ptr(), tb, ignore_index, (float)scale,
                                  static_cast<float*>(loss.data_ptr()), static_cast<float*>(tw.data_ptr()),
                                  static_cast<float*>(ptr(lse)), flag_ptr(flag), wsp.data_ptr(), ws_bytes,
                                  stream_of(logits)));
  return return_lse ? py::make_tuple(loss, tw, lse) : py::make_tuple(loss, tw);
}

py::object cross_entropy_forward_backward(const Tensor& logits, const py::object& targets, double grad_loss,
                                          int64_t ignore_index, double scale, bool return_loss, bool in_place,
                                          const std::optional<Tensor>& flag) {
  need_gpu("cross_entropy logits", logits);
  const auto dev = logits.device();
  const int64_t V = logits.dim() ? logits.size(-1) : 1;
  Rows l = as_rows(logits, V);
  int tb = 0;
  Tensor t = targets_of(targets, l.m, dev, tb);
  Tensor out;
  if (in_place) {
    if (!logits.is_contiguous()) fail("cross_entropy_forward_backward: in_place needs contiguous logits");
    out = logits;
  } else {
    out = at::empty(logits.sizes(), logits.options().dtype(at::kBFloat16));
  }
  Tensor loss, tw, wsp;
  size_t ws_bytes = 0;
  if (return_loss) {
    const auto f32 = logits.options().dtype(at::kFloat);
    loss = at::empty({}, f32);
    tw = at::empty({}, f32);
    ws_bytes = kp_cross_entropy_fwd_workspace_size(l.m);
    wsp = at::empty({(int64_t)std::max<size_t>(ws_bytes, 8)}, logits.options().dtype(at::kByte));
  }
  check("kp_cross_entropy_fwd_bwd_bf16",
        kp_cross_entropy_fwd_bwd_bf16(l.t.data_ptr(), l.stride, l.m, V, t.data_ptr(), tb, ignore_index,
                                      (float)grad_loss, out.data_ptr(), V, (float)scale,
                                      static_cast<float*>(ptr(loss)), static_cast<float*>(ptr(tw)), flag_ptr(flag),
                                      ptr(wsp), ws_bytes, stream_of(logits)));
  if (return_loss) return py::make_tuple(out, loss, tw);
  return py::cast(out);
}

Tensor cross_entropy_backward(const Tensor& log_softmax, const py::object& targets, double grad_loss,
                              int64_t ignore_index, const std::optional<Tensor>& flag) {
  need_gpu("cross_entropy log_softmax", log_softmax, at::kFloat);
  const auto dev = log_softmax.device();
  const int64_t V = log_softmax.dim() ? log_softmax.size(-1) : 1;
  Rows l = as_rows(log_softmax, V);
  int tb = 0;
  Tensor t = targets_of(targets, l.m, dev, tb);
  Tensor out = at::empty(log_softmax.sizes(), log_softmax.options().dtype(at::kBFloat16));
  if (l.m)
    check("kp_cross_entropy_bwd_bf16",
          kp_cross_entropy_bwd_bf16(static_cast<const float*>(l.t.data_ptr()), l.stride, t.data_ptr(), tb,
                                    ignore_index, (float)grad_loss, out.data_ptr(), V, l.m, V, flag_ptr(flag),
                                    stream_of(log_softmax)));
  return out;
}

// -------------------------------------------------------------------- RoPE
// A [B, S, H, D] operand with unit stride on D (copied if not): its strides
// over B, S and H.
Tensor rope_operand(Tensor t, const char* who, int64_t st[3]) {
  if (t.dim() != 4) fail(std::string(who) + ": expected [B, S, H, D], got shape " + shape_str(t.sizes()));
  if (t.size(3) > 1 && t.stride(3) != 1) t = t.contiguous();
  for (int i = 0; i < 3; ++i) st[i] = t.stride(i);
  return t;
}

struct Positions {
  const void* p = nullptr;
  int bytes = 0;
  int64_t sb = 0, ss = 0;
};
Positions positions_of(const std::optional<Tensor>& positions, int64_t B, int64_t S, const at::Device& dev,
                       const std::string& who) {
  Positions r;
  if (!positions) return r;
  const Tensor& p = *positions;
  if (p.device() != dev || (p.scalar_type() != at::kInt && p.scalar_type() != at::kLong))
    fail(who + ": positions must be an int32/int64 tensor on the same device");
  if (p.dim() == 1) {
    if (p.size(0) != S) fail(who + ": 1-D positions must have S entries");
    r.sb = 0;
    r.ss = p.stride(0);
  } else if (p.dim() == 2) {
    if (p.size(1) != S || (p.size(0) != 1 && p.size(0) != B)) fail(who + ": 2-D positions must be [B, S] or [1, S]");
    r.sb = p.size(0) == B ? p.stride(0) : 0;
    r.ss = p.stride(1);
  } else {
    fail(who + ": positions must be 1-D or 2-D");
  }
  r.p = p.data_ptr();
  r.bytes = (int)p.element_size();
  return r;
}

py::tuple rope(Tensor q, std::optional<Tensor> k, const std::optional<Tensor>& positions, std::optional<double> theta,
               const std::optional<Tensor>& freqs_cis, int64_t mode, bool conj, bool q_f32, bool k_f32, bool copies,
               const std::optional<Tensor>& flag) {
  need_gpu("rope q", q);
  const auto dev = q.device();
  int64_t qs[3], ks[3] = {0, 0, 0};
  q = rope_operand(q, "rope", qs);
  const int64_t B = q.size(0), S = q.size(1), Hq = q.size(2), D = q.size(3);
  const auto opts = q.options();
  Tensor q_out = at::empty({B, S, Hq, D}, opts.dtype(q_f32 ? at::kFloat : at::kBFloat16));
  Tensor kk, k_out;
  if (k) {
    need_gpu("rope k", *k);
    kk = rope_operand(*k, "rope", ks);
    if (kk.size(0) != B || kk.size(1) != S || kk.size(3) != D) fail("rope: q and k must agree on B, S and D");
    k_out = at::empty(kk.sizes(), opts.dtype(k_f32 ? at::kFloat : at::kBFloat16));
  }
  const Positions pos = positions_of(positions, B, S, dev, "rope");
  const float* f_ptr = nullptr;
  int64_t frows = 0, frs = 0;
  double th = 0.0;
  Tensor fc;
  if (freqs_cis) {
    const Tensor& f = *freqs_cis;
    if (f.device() != dev || f.scalar_type() != at::kComplexFloat)
      fail("rope: freqs_cis must be complex64 on the same device");
    if (f.size(-1) != D / 2) fail("rope: freqs_cis last dim must be D/2=" + std::to_string(D / 2));
    Rows r = as_rows(f, D / 2);
    fc = r.t;
    frs = r.stride;
    frows = r.m;
    f_ptr = static_cast<const float*>(fc.data_ptr());
  } else {
    if (!theta || !(*theta > 0) || !std::isfinite(*theta)) fail("rope: need theta > 0 or freqs_cis");
    th = *theta;
  }
  int64_t qos[3] = {q_out.stride(0), q_out.stride(1), q_out.stride(2)};
  int64_t kos[3] = {0, 0, 0};
  if (k_out.defined())
    for (int i = 0; i < 3; ++i) kos[i] = k_out.stride(i);
  const int mask = (q_f32 ? 1 : 0) | (k_out.defined() && k_f32 ? 2 : 0);
  int32_t* fl = flag_ptr(flag);
  const DeviceStream s = stream_of(q);  // the device stays current to the end of the function
  if (copies) {
    Tensor q_copy = at::empty_like(q_out);
    Tensor k_copy = k_out.defined() ? at::empty_like(k_out) : Tensor();
    check("kp_rope_bf16_twice",
          kp_rope_bf16_twice(q.data_ptr(), q_out.data_ptr(), Hq, qs, qos, ptr(kk), ptr(k_out),
                             kk.defined() ? kk.size(2) : 0, kk.defined() ? ks : nullptr,
                             k_out.defined() ? kos : nullptr, B, S, D, pos.p, pos.bytes, pos.sb, pos.ss, (int)mode, th,
                             f_ptr, frows, frs, conj ? 1 : 0, mask, q_copy.data_ptr(), ptr(k_copy), fl, s));
    return py::make_tuple(q_out, opt(k_out), q_copy, opt(k_copy));
  }
  check("kp_rope_bf16", kp_rope_bf16(q.data_ptr(), q_out.data_ptr(), Hq, qs, qos, ptr(kk), ptr(k_out),
                                     kk.defined() ? kk.size(2) : 0, kk.defined() ? ks : nullptr,
                                     k_out.defined() ? kos : nullptr, B, S, D, pos.p, pos.bytes, pos.sb, pos.ss,
                                     (int)mode, th, f_ptr, frows, frs, conj ? 1 : 0, mask, fl, s));
  return py::make_tuple(q_out, opt(k_out));
}

py::tuple rope_complex(Tensor q, std::optional<Tensor> k, const Tensor& freqs_cis,
                       const std::optional<Tensor>& positions, bool conj, const std::optional<Tensor>& flag) {
  need_gpu("rope_complex q", q, at::kComplexFloat);
  const auto dev = q.device();
  if (q.dim() != 4) fail("rope_complex: expected [B, S, H, P], got shape " + shape_str(q.sizes()));
  if (q.size(3) > 1 && q.stride(3) != 1) q = q.contiguous();
  const int64_t B = q.size(0), S = q.size(1), Hq = q.size(2), P = q.size(3);
  const auto opts = q.options().dtype(at::kComplexFloat);
  Tensor q_out = at::empty(q.sizes(), opts);
  Tensor kk, k_out;
  int64_t ks[3] = {0, 0, 0}, kos[3] = {0, 0, 0};
  if (k) {
    need_gpu("rope_complex k", *k, at::kComplexFloat);
    kk = *k;
    if (kk.dim() != 4 || kk.size(0) != B || kk.size(1) != S || kk.size(3) != P)
      fail("rope_complex: q and k must agree on B, S and P");
    if (kk.size(3) > 1 && kk.stride(3) != 1) kk = kk.contiguous();
    k_out = at::empty(kk.sizes(), opts);
    for (int i = 0; i < 3; ++i) {
      ks[i] = kk.stride(i);
      kos[i] = k_out.stride(i);
    }
  }
  if (freqs_cis.device() != dev || freqs_cis.scalar_type() != at::kComplexFloat || freqs_cis.size(-1) != P)
    fail("rope_complex: freqs_cis must be complex64 on the same device with last dim " + std::to_string(P));
  Rows f = as_rows(freqs_cis, P);
  const Positions pos = positions_of(positions, B, S, dev, "rope");
  if (B * S) {
    int64_t qs[3] = {q.stride(0), q.stride(1), q.stride(2)};
    int64_t qos[3] = {q_out.stride(0), q_out.stride(1), q_out.stride(2)};
    check("kp_rope_c64",
          kp_rope_c64(q.data_ptr(), q_out.data_ptr(), Hq, qs, qos, ptr(kk), ptr(k_out), kk.defined() ? kk.size(2) : 0,
                      kk.defined() ? ks : nullptr, k_out.defined() ? kos : nullptr, B, S, P, pos.p, pos.bytes, pos.sb,
                      pos.ss, static_cast<const float*>(f.t.data_ptr()), f.m, f.stride, conj ? 1 : 0,
                      flag_ptr(flag), stream_of(q)));
  }
  return py::make_tuple(q_out, opt(k_out));
}

}  // namespace

PYBIND11_MODULE(_kp_torch, m) {
  m.doc() = "Native tensor-level wrappers of libkp_hip.so's entry points (kernelproblems_amd.fused)";
  m.def("rms_norm", &rms_norm);
  m.def("rms_norm_backward", &rms_norm_backward);
  m.def("rms_norm_forward_backward", &rms_norm_forward_backward);
  m.def("embedding", &embedding);
  m.def("embedding_rms_norm", &embedding_rms_norm);
  m.def("embedding_dense_backward", &embedding_dense_backward);
  m.def("rms_norm_embedding_backward", &rms_norm_embedding_backward);
  m.def("rope", &rope);
  m.def("rope_complex", &rope_complex);
  m.def("unshard", &unshard);
  m.def("swiglu", &swiglu);
  m.def("swiglu_backward", &swiglu_backward);
  m.def("silu", &silu);
  m.def("swiglu_forward_backward", &swiglu_forward_backward);
  m.def("cross_entropy_loss", &cross_entropy_loss);
  m.def("cross_entropy_forward_backward", &cross_entropy_forward_backward);
  m.def("cross_entropy_backward", &cross_entropy_backward);
}
