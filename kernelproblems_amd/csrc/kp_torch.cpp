// Native tensor-level wrappers of the most-called entry points of
// kernelproblems_amd.fused: rms_norm, rms_norm_backward, embedding, rope and
// rope_complex.  Each does what the Python wrapper did -- check the tensors,
// find the row layout, allocate outputs and workspace with torch's caching
// allocator, and call the C ABI (include/kp.h) on the device's current stream --
// in one native call, so that a drop-in's host time per call is the kernel
// launches plus a few allocations rather than Python argument marshalling
// (a small fragment's kernel runs for less time than that marshalling took).
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

void* stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void* ptr(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

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

py::tuple rms_norm_backward(const std::vector<Tensor>& dy_terms, const std::vector<Tensor>& x_terms,
                            const std::optional<Tensor>& rstd, const std::optional<Tensor>& weight, double eps,
                            int64_t n, const std::optional<Tensor>& dx_residual, bool want_dx,
                            const std::optional<std::string>& dw) {
  static const char* who = "rms_norm_backward";
  const std::string w_ = who;
  if (dy_terms.empty() || dy_terms.size() > 3 || x_terms.empty() || x_terms.size() > 3)
    fail(w_ + ": 1..3 grad terms and 1..3 input terms");
  const Tensor& dy0 = dy_terms[0];
  need_gpu(w_ + " grad_out", dy0);
  const auto shape = x_terms[0].sizes();
  Tensor dyr[3], xr[3];
  const void* dyp[3];
  const void* xp[3];
  int64_t dys[3], xs[3];
  int64_t m = 0;
  for (size_t i = 0; i < dy_terms.size(); ++i) {
    const Tensor& t = dy_terms[i];
    need_gpu(w_ + " grad term " + std::to_string(i), t);
    if (t.numel() != dy0.numel()) fail(w_ + ": grad terms must have the same number of elements");
    Rows r = as_rows(t, n);
    dyr[i] = r.t;
    dyp[i] = r.t.data_ptr();
    dys[i] = r.stride;
    m = r.m;
  }
  for (size_t i = 0; i < x_terms.size(); ++i) {
    const Tensor& t = x_terms[i];
    need_gpu(w_ + " input term " + std::to_string(i), t);
    if (t.numel() != dy0.numel()) fail(w_ + ": input and grad must have the same number of elements");
    Rows r = as_rows(t, n);
    xr[i] = r.t;
    xp[i] = r.t.data_ptr();
    xs[i] = r.stride;
  }
  Segments ws{Tensor(), n, n};
  if (weight) {
    need_gpu(w_ + " weight", *weight);
    ws = weight_segments(*weight, n);
  }
  Tensor res;
  int64_t res_s = n;
  if (dx_residual) {
    need_gpu(w_ + " residual", *dx_residual);
    Rows r = as_rows(*dx_residual, n);
    res = r.t;
    res_s = r.stride;
  }
  Tensor rstd_t;
  if (rstd) {
    need_gpu(w_ + " rstd", *rstd, at::kFloat);
    if (rstd->numel() != m)
      fail(w_ + ": rstd has " + std::to_string(rstd->numel()) + " values, expected " + std::to_string(m));
    rstd_t = rstd->contiguous();
  }
  const auto bf = dy0.options().dtype(at::kBFloat16);
  Tensor dx = at::empty(shape, bf);
  Tensor dw_f32, dw_bf16;
  if (dw) {
    if (!weight) fail(w_ + ": no weight, no weight gradient");
    if (*dw == "f32" || *dw == "f32_bf16") dw_f32 = at::empty({n}, bf.dtype(at::kFloat));
    else if (*dw == "bf16") dw_bf16 = at::empty({n}, bf);
    else throw py::value_error(w_ + ": unknown dw mode '" + *dw + "'");
  }
  size_t ws_bytes = 0;
  Tensor wsp;
  if (dw) {
    ws_bytes = kp_rmsnorm_bwd_workspace_size(m, n);
    wsp = at::empty({(int64_t)std::max<size_t>(ws_bytes, 16)}, bf.dtype(at::kByte));
  }
  check("kp_rmsnorm_bwd_bf16",
        kp_rmsnorm_bwd_bf16(dyp, dys, (int)dy_terms.size(), xp, xs, (int)x_terms.size(),
                            static_cast<const float*>(ptr(rstd_t)), ptr(ws.w), ws.len, ws.stride, ptr(res), res_s,
                            dx.data_ptr(), n, static_cast<float*>(ptr(dw_f32)), ptr(dw_bf16),
                            (dw && *dw == "f32_bf16") ? 1 : 0, m, n, (float)eps, ptr(wsp), ws_bytes,
                            stream_of(dy0)));
  Tensor out_dw = dw_f32.defined() ? dw_f32 : dw_bf16;
  if (weight && out_dw.defined()) out_dw = out_dw.view(weight->sizes());
  return py::make_tuple(want_dx ? py::cast(dx) : py::none(), opt(out_dw));
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
                              flag ? static_cast<int32_t*>(flag->data_ptr()) : nullptr, stream_of(table)));
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
  int32_t* fl = flag ? static_cast<int32_t*>(flag->data_ptr()) : nullptr;
  void* s = stream_of(q);
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
                      flag ? static_cast<int32_t*>(flag->data_ptr()) : nullptr, stream_of(q)));
  }
  return py::make_tuple(q_out, opt(k_out));
}

}  // namespace

PYBIND11_MODULE(_kp_torch, m) {
  m.doc() = "Native tensor-level wrappers of libkp_hip.so's hottest entry points";
  m.def("rms_norm", &rms_norm);
  m.def("rms_norm_backward", &rms_norm_backward);
  m.def("embedding", &embedding);
  m.def("rope", &rope);
  m.def("rope_complex", &rope_complex);
}
