// Torch binding of libmhc_hip for MHCLayer's hot calls (mhc_mlx/layer.py:339-435).
//
// The module's work per call is one or two library launches; at small batch
// its latency is the host code around them.  This binding does that host code
// in C++ over the same C ABI (include/mhc_hip.h): the layer's autograd
// Function (forward: Sinkhorn projection + fused kernel; backward: partial
// sums, fixed-order reduction, Sinkhorn VJP) and the no-gradient forward.
// The backward therefore runs on the autograd engine's thread without Python.
// Every launch goes to the current HIP stream of the input's device, as the
// Python wrappers' do; arguments are validated by the Python caller
// (mhc_mlx_amd/ops.py), and the library checks its own again.
#include <torch/extension.h>

#include <cstdlib>

#include <c10/hip/HIPStream.h>
#include <torch/csrc/Dtype.h>
#include <torch/csrc/autograd/python_variable.h>

#include "mhc_hip.h"

namespace {

using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return MHC_DTYPE_F32;
    case at::kBFloat16: return MHC_DTYPE_BF16;
    case at::kHalf: return MHC_DTYPE_F16;
    default: TORCH_CHECK_VALUE(false, "unsupported dtype ", t, "; expected float32, bfloat16 or float16");
  }
}

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.get_device()).stream(); }

// Library status -> exception: a rejected argument is a ValueError, a HIP
// failure a RuntimeError (the Python wrappers' convention).
void check(int rc, const char* what) {
  if (rc == MHC_OK) return;
  const char* msg = mhc_last_error();
  TORCH_CHECK_VALUE(rc > 0, what, ": ", msg ? msg : "invalid argument");
  TORCH_CHECK(false, what, " failed (hip error ", rc, "): ", msg ? msg : "");
}

at::Tensor f32(const at::Tensor& t) {
  return t.scalar_type() == at::kFloat && t.is_contiguous() ? t : t.to(at::kFloat).contiguous();
}

// x [T, n, C] and the parameters on x's GPU (the kernels take raw device
// pointers) with the element counts the kernels read: [n], [n], [n, n], [C],
// or [T, n], [T, n], [T, n, n] per token.
void check_inputs(const at::Tensor& x, const at::Tensor& hpre, const at::Tensor& hpost, const at::Tensor& hres,
                  const at::Tensor& w, bool per_token) {
  TORCH_CHECK_VALUE(x.dim() == 3, "x must be [B, n, C], got ", x.sizes());
  TORCH_CHECK_VALUE(x.is_cuda(), "the HIP path needs GPU tensors (got x on ", x.device(), ")");
  for (const at::Tensor* p : {&hpre, &hpost, &hres, &w})
    TORCH_CHECK_VALUE(p->device() == x.device(), "parameters must be on x's device ", x.device(), " (got ",
                      p->device(), ")");
  const int64_t T = x.size(0), n = x.size(1), C = x.size(2), k = per_token ? T : 1;
  TORCH_CHECK_VALUE(hpre.numel() == k * n && hpost.numel() == k * n && hres.numel() == k * n * n &&
                        w.numel() == C,
                    "parameter sizes do not match x ", x.sizes());
}

float* fp(const at::Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }

// mhc_layer_fwd: out [T, n, C] of out_dtype and M (Sinkhorn of the logits,
// [n, n] or [T, n, n]); with `state` defined, the projection also records its
// VJP state there (mhc_sinkhorn_fwd_record + mhc_fused_fwd).
std::pair<at::Tensor, at::Tensor> layer_fwd(const at::Tensor& x, const at::Tensor& hp, const at::Tensor& hq,
                                            const at::Tensor& hr, const at::Tensor& w, int64_t iters, double eps,
                                            at::ScalarType out_dtype, bool per_token, const at::Tensor& state) {
  const int64_t T = x.size(0);
  const int n = (int)x.size(1), C = (int)x.size(2);
  at::Tensor out = at::empty({T, n, C}, x.options().dtype(out_dtype));
  at::Tensor M = at::empty_like(hr);
  void* s = stream_of(x);
  if (!state.defined()) {
    check(mhc_layer_fwd(x.data_ptr(), dtype_code(x.scalar_type()), fp(hp), fp(hq), fp(hr), fp(w), out.data_ptr(),
                        dtype_code(out_dtype), fp(M), T, n, C, per_token ? 1 : 0, (int)iters, (float)eps, s),
          "mhc_layer_fwd");
    return {out, M};
  }
  check(mhc_sinkhorn_fwd_record(fp(hr), fp(M), state.data_ptr(), (size_t)state.numel(), per_token ? T : 1, n,
                                (int)iters, (float)eps, s),
        "mhc_sinkhorn_fwd_record");
  check(mhc_fused_fwd(x.data_ptr(), dtype_code(x.scalar_type()), fp(M), per_token ? (int64_t)n * n : 0, fp(hp),
                      fp(hq), per_token ? n : 0, MHC_H_RAW, fp(w), out.data_ptr(), dtype_code(out_dtype), nullptr, T,
                      n, C, (float)eps, s),
        "mhc_fused_fwd");
  return {out, M};
}

// layer_fwd (layer-wide parameters, no record) for a call that needs no
// gradient: out and the projection M share one allocation (out first, M at
// the next 256-byte boundary), since only out is returned and one allocation
// costs less host time than two.  out is a view of the whole buffer's first
// T*n*C elements.
at::Tensor layer_fwd_nograd(const at::Tensor& x, const at::Tensor& hp, const at::Tensor& hq, const at::Tensor& hr,
                            const at::Tensor& w, int64_t iters, double eps, at::ScalarType out_dtype) {
  const int64_t T = x.size(0);
  const int n = (int)x.size(1), C = (int)x.size(2);
  const int64_t elt = (int64_t)c10::elementSize(out_dtype), nout = T * n * C;
  const int64_t m_off = (nout * elt + 255) / 256 * 256;  // bytes
  const int64_t total = (m_off + (int64_t)n * n * 4 + elt - 1) / elt;
  at::Tensor buf = at::empty({total}, x.options().dtype(out_dtype));
  float* M = reinterpret_cast<float*>(static_cast<char*>(buf.data_ptr()) + m_off);
  check(mhc_layer_fwd(x.data_ptr(), dtype_code(x.scalar_type()), fp(hp), fp(hq), fp(hr), fp(w), buf.data_ptr(),
                      dtype_code(out_dtype), M, T, n, C, 0, (int)iters, (float)eps, stream_of(x)),
        "mhc_layer_fwd");
  return buf.narrow(0, 0, nout).view({T, n, C});
}

// VJP of layer_fwd: (dx, dH_pre_raw, dH_post_raw, dH_res_raw, d_rms_weight).
variable_list layer_bwd(const at::Tensor& x, const at::Tensor& g_in, const at::Tensor& hp, const at::Tensor& hq,
                        const at::Tensor& hr, const at::Tensor& M, const at::Tensor& w, int64_t iters, double eps,
                        bool per_token, const at::Tensor& state) {
  const int64_t T = x.size(0);
  const int n = (int)x.size(1), C = (int)x.size(2);
  const at::ScalarType gt = g_in.scalar_type() == at::kFloat || g_in.scalar_type() == x.scalar_type()
                                ? g_in.scalar_type() : at::kFloat;
  at::Tensor g = g_in.scalar_type() == gt ? g_in : g_in.to(gt);
  if (!g.is_contiguous()) g = g.contiguous();
  at::Tensor dx = at::empty_like(x);
  // the four parameter gradients as views of one allocation (each contiguous with the parameter's shape,
  // starting on a 256-byte boundary as a separate allocation would)
  auto up = [](int64_t v) { return (v + 63) / 64 * 64; };
  const int64_t o1 = up(hp.numel()), o2 = o1 + up(hq.numel()), o3 = o2 + up(hr.numel());
  at::Tensor pg = at::empty({o3 + C}, w.options());
  at::Tensor dpre = pg.narrow(0, 0, hp.numel()).view(hp.sizes());
  at::Tensor dpost = pg.narrow(0, o1, hq.numel()).view(hq.sizes());
  at::Tensor dres = pg.narrow(0, o2, hr.numel()).view(hr.sizes());
  at::Tensor dw = pg.narrow(0, o3, C);
  const int xc = dtype_code(x.scalar_type()), gc = dtype_code(gt);
  void* s = stream_of(x);
  const int pt = per_token ? 1 : 0;
  if (!state.defined()) {
    const size_t nb = mhc_layer_bwd_workspace_bytes(T, n, C, pt, (int)iters);
    at::Tensor ws = at::empty({(int64_t)std::max<size_t>(nb, 1)}, x.options().dtype(at::kByte));
    check(mhc_layer_bwd(x.data_ptr(), xc, g.data_ptr(), gc, fp(hp), fp(hq), fp(hr), fp(M), fp(w), dx.data_ptr(),
                        fp(dpre), fp(dpost), fp(dres), fp(dw), ws.data_ptr(), nb, T, n, C, pt, (int)iters, (float)eps,
                        s),
          "mhc_layer_bwd");
    return {dx, dpre, dpost, dres, dw};
  }
  // from the recorded Sinkhorn state: partial sums (per token: dM of each token into dres, the activated-H
  // chain applied in the kernel), the reduction, then the recorded VJP (in place per token)
  at::Tensor dM = per_token ? dres : at::empty({n, n}, hr.options());
  const size_t nb = mhc_fused_bwd_workspace_bytes(T, n, C, pt);
  at::Tensor ws = at::empty({(int64_t)std::max<size_t>(nb, 1)}, x.options().dtype(at::kByte));
  int64_t np = 0;
  check(mhc_fused_bwd_partials(x.data_ptr(), xc, g.data_ptr(), gc, fp(M), pt ? (int64_t)n * n : 0, fp(hp), fp(hq),
                               pt ? n : 0, MHC_H_RAW, fp(w), dx.data_ptr(), xc, pt ? fp(dres) : nullptr,
                               pt ? fp(dpre) : nullptr, pt ? fp(dpost) : nullptr, ws.data_ptr(), nb, T, n, C,
                               (float)eps, &np, s),
        "mhc_fused_bwd_partials");
  check(mhc_reduce_param_grads(ws.data_ptr(), nb, np, n, C, pt, pt ? nullptr : fp(hp), pt ? nullptr : fp(hq),
                               MHC_H_RAW, pt ? nullptr : fp(dM), pt ? nullptr : fp(dpre), pt ? nullptr : fp(dpost),
                               fp(dw), s),
        "mhc_reduce_param_grads");
  check(mhc_sinkhorn_bwd_recorded(fp(hr), fp(dM), fp(dres), state.data_ptr(), (size_t)state.numel(), pt ? T : 1, n,
                                  (int)iters, (float)eps, s),
        "mhc_sinkhorn_bwd_recorded");
  return {dx, dpre, dpost, dres, dw};
}

// MHCLayer forward/backward from raw parameters, as an autograd Function.
// Inputs as the library takes them: x contiguous (fp32 / bf16 / fp16),
// parameters fp32 contiguous on x's device.  With `record` the Sinkhorn
// projection records its VJP state (n = 16 per token, 16 < n <= 64) when
// the library has a recorded path for n.
struct LayerFn : public torch::autograd::Function<LayerFn> {
  static at::Tensor forward(AutogradContext* ctx, const at::Tensor& x, const at::Tensor& hpre,
                            const at::Tensor& hpost, const at::Tensor& hres, const at::Tensor& w, int64_t iters,
                            double eps, int64_t out_code, bool per_token, bool record) {
    const at::ScalarType out_dtype = out_code == MHC_DTYPE_BF16 ? at::kBFloat16
                                     : out_code == MHC_DTYPE_F16 ? at::kHalf : at::kFloat;
    at::Tensor state;
    // (the n = 16 batched kernels read 16-byte aligned logits: an offset view is projected without a record)
    if (record && x.size(0) > 0 && (x.size(1) != 16 || reinterpret_cast<uintptr_t>(hres.data_ptr()) % 16 == 0)) {
      const size_t nst = mhc_sinkhorn_state_bytes(per_token ? x.size(0) : 1, (int)x.size(1), (int)iters);
      if (nst > 0) state = at::empty({(int64_t)nst}, x.options().dtype(at::kByte));
    }
    auto r = layer_fwd(x, hpre, hpost, hres, w, iters, eps, out_dtype, per_token, state);
    ctx->save_for_backward({x, hpre, hpost, hres, w, r.second, state});
    ctx->saved_data["iters"] = iters;
    ctx->saved_data["eps"] = eps;
    ctx->saved_data["per_token"] = per_token;
    return r.first;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto sv = ctx->get_saved_variables();
    variable_list g = layer_bwd(sv[0], grads[0], sv[1], sv[2], sv[3], sv[5], sv[4], ctx->saved_data["iters"].toInt(),
                                ctx->saved_data["eps"].toDouble(), ctx->saved_data["per_token"].toBool(), sv[6]);
    return {g[0], g[1], g[2], g[3], g[4], at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor(), at::Tensor()};
  }
};

// Autograd entry: parameters are converted to contiguous fp32 here (a no-op
// when they already are), with the conversion inside the autograd graph so
// gradients reach the caller's tensors in their own dtype.
at::Tensor layer_apply(const at::Tensor& x, const at::Tensor& hpre, const at::Tensor& hpost, const at::Tensor& hres,
                       const at::Tensor& w, int64_t iters, double eps, int64_t out_code, bool per_token, bool record) {
  check_inputs(x, hpre, hpost, hres, w, per_token);
  return LayerFn::apply(x.contiguous(), f32(hpre), f32(hpost), f32(hres), f32(w), iters, eps, out_code, per_token,
                        record);
}

// The forward of a call that needs no gradient: out only.
at::Tensor layer_forward_nograd(const at::Tensor& x, const at::Tensor& hpre, const at::Tensor& hpost,
                                const at::Tensor& hres, const at::Tensor& w, int64_t iters, double eps,
                                int64_t out_code, bool per_token) {
  check_inputs(x, hpre, hpost, hres, w, per_token);
  const at::ScalarType out_dtype = out_code == MHC_DTYPE_BF16 ? at::kBFloat16
                                   : out_code == MHC_DTYPE_F16 ? at::kHalf : at::kFloat;
  if (!per_token) return layer_fwd_nograd(x.contiguous(), f32(hpre), f32(hpost), f32(hres), f32(w), iters, eps, out_dtype);
  return layer_fwd(x.contiguous(), f32(hpre), f32(hpost), f32(hres), f32(w), iters, eps, out_dtype, per_token,
                   at::Tensor()).first;
}

bool env_is_one(const char* name) {
  const char* v = std::getenv(name);
  return v != nullptr && v[0] == '1' && v[1] == '\0';
}

// MHCLayer's forward on the accelerated path, all of its host steps in one
// call (mhc_mlx/layer.py:339-435): an undefined tensor (None in Python) when
// MHC_MLX_DISABLE_METAL=1 or MHC_HIP_DISABLE=1 is set (read per call through
// getenv, which sees os.environ's changes, as the reference reads its switch
// per call, layer.py:176) or when the call is not one this path takes (x not
// [B, n, C] for the layer's n and C, tensors off x's GPU, n > 64, a dtype the
// kernels do not read), so that the module's general path decides and raises
// the reference's errors.  Otherwise the output: the kernel writes
// return_dtype directly when it is x's half type (layer.py:361-364), else fp32
// cast to return_dtype; the autograd node is recorded when grad mode is on and
// x or a parameter requires a gradient.
at::Tensor module_forward(const at::Tensor& x, const at::Tensor& hpre, const at::Tensor& hpost,
                          const at::Tensor& hres, const at::Tensor& w, int64_t n, int64_t C, int64_t iters,
                          double eps, c10::optional<at::ScalarType> return_dtype) {
  if (env_is_one("MHC_MLX_DISABLE_METAL") || env_is_one("MHC_HIP_DISABLE")) return at::Tensor();
  if (n < 1 || n > MHC_MAX_N || x.dim() != 3 || x.size(1) != n || x.size(2) != C || !x.is_cuda()) return at::Tensor();
  const at::ScalarType xt = x.scalar_type();
  if (xt != at::kFloat && xt != at::kBFloat16 && xt != at::kHalf) return at::Tensor();
  const at::Device dev = x.device();
  for (const at::Tensor* p : {&hpre, &hpost, &hres, &w})
    if (p->device() != dev) return at::Tensor();
  if (hpre.numel() != n || hpost.numel() != n || hres.numel() != n * n || w.numel() != C) return at::Tensor();
  const bool half_out = return_dtype.has_value() && *return_dtype == xt && xt != at::kFloat;
  const int64_t code = half_out ? dtype_code(xt) : MHC_DTYPE_F32;
  at::Tensor out;
  if (at::GradMode::is_enabled() && (x.requires_grad() || hpre.requires_grad() || hpost.requires_grad() ||
                                     hres.requires_grad() || w.requires_grad())) {
    out = LayerFn::apply(x.contiguous(), f32(hpre), f32(hpost), f32(hres), f32(w), iters, eps, code, false, n > 16);
  } else {
    out = layer_fwd_nograd(x.contiguous(), f32(hpre), f32(hpost), f32(hres), f32(w), iters, eps,
                           half_out ? xt : at::kFloat);
  }
  if (return_dtype.has_value() && out.scalar_type() != *return_dtype) out = out.to(*return_dtype);
  return out;
}

// module_forward called with the module itself: its parameters, n, C,
// sinkhorn_iters, eps and use_metal are read from the instance dict here, so
// one call with three arguments carries MHCLayer.forward's whole fast path.
// Anything unexpected there (a deleted or replaced-by-None parameter, an
// attribute of another type) leaves the call to the general path.
at::Tensor module_call(py::handle mod, py::handle x_obj, py::handle rd_obj) {
  py::object dict_obj = py::reinterpret_steal<py::object>(PyObject_GetAttrString(mod.ptr(), "__dict__"));
  if (!dict_obj) {
    PyErr_Clear();
    return at::Tensor();
  }
  PyObject* d = dict_obj.ptr();
  if (!PyDict_Check(d) || PyDict_GetItemString(d, "use_metal") != Py_True) return at::Tensor();
  PyObject* ps = PyDict_GetItemString(d, "_parameters");
  PyObject* n_obj = PyDict_GetItemString(d, "n");
  PyObject* c_obj = PyDict_GetItemString(d, "C");
  PyObject* it_obj = PyDict_GetItemString(d, "sinkhorn_iters");
  PyObject* eps_obj = PyDict_GetItemString(d, "eps");
  if (ps == nullptr || !PyDict_Check(ps) || n_obj == nullptr || !PyLong_Check(n_obj) || c_obj == nullptr ||
      !PyLong_Check(c_obj) || it_obj == nullptr || !PyLong_Check(it_obj) || eps_obj == nullptr ||
      !PyFloat_Check(eps_obj) || !THPVariable_Check(x_obj.ptr()))
    return at::Tensor();
  PyObject* t[4] = {PyDict_GetItemString(ps, "H_pre_raw"), PyDict_GetItemString(ps, "H_post_raw"),
                    PyDict_GetItemString(ps, "H_res_raw"), PyDict_GetItemString(ps, "rms_weight")};
  for (PyObject* o : t)
    if (o == nullptr || !THPVariable_Check(o)) return at::Tensor();
  c10::optional<at::ScalarType> rd;
  if (rd_obj.ptr() != Py_None) {
    if (!THPDtype_Check(rd_obj.ptr())) return at::Tensor();
    rd = reinterpret_cast<THPDtype*>(rd_obj.ptr())->scalar_type;
  }
  const long long n = PyLong_AsLongLong(n_obj), C = PyLong_AsLongLong(c_obj), iters = PyLong_AsLongLong(it_obj);
  if (PyErr_Occurred()) {
    PyErr_Clear();
    return at::Tensor();
  }
  return module_forward(THPVariable_Unpack(x_obj.ptr()), THPVariable_Unpack(t[0]), THPVariable_Unpack(t[1]),
                        THPVariable_Unpack(t[2]), THPVariable_Unpack(t[3]), n, C, iters,
                        PyFloat_AS_DOUBLE(eps_obj), rd);
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "torch binding of libmhc_hip for MHCLayer's forward and backward";
  m.def("layer_apply", &layer_apply, "MHCLayer forward with its backward as a C++ autograd Function");
  m.def("layer_forward_nograd", &layer_forward_nograd, "MHCLayer forward without autograd");
  m.def("module_forward", &module_forward, "MHCLayer.forward's accelerated path (None: take the general path)");
  m.def("module_call", &module_call, "module_forward with the arguments read from the MHCLayer instance");
}
