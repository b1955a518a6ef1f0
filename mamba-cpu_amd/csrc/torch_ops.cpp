// The mamba_cpu torch operators, in C++ over the C ABI of libmamba_hip.so.
//
// Same operator names and schemas as the reference's Python custom ops
// (src/mamba_cpu/ops/selective_scan_interface.py:16-124,
// src/mamba_cpu/ops/causal_conv1d.py, src/mamba_cpu/ops/selective_state_update.py),
// registered for the CUDA dispatch key (ROCm GPU tensors), with their autograd
// formulas registered for the Autograd key as torch::autograd::Functions. The
// bodies check their arguments (ValueError / NotImplementedError, as the
// reference raises), allocate outputs and workspaces through the torch caching
// allocator and launch on the current stream; they never synchronise.
// Fake (meta) implementations are registered from Python, next to the public
// functions (mamba_cpu/ops/*.py).
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include <algorithm>
#include <cstring>
#include <limits>
#include <optional>
#include <tuple>

#include <rocblas/rocblas.h>

#include "mamba_hip.h"

namespace mcpu_torch {
namespace {

using at::Tensor;
using std::optional;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

// ---- helpers ------------------------------------------------------------------

void* stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_rc(int rc, const char* what) {
  if (rc == MCPU_OK) return;
  const char* msg = mcpu_last_error();
  TORCH_CHECK_VALUE(rc != MCPU_ERR_INVALID, what, ": ", msg);
  TORCH_CHECK_NOT_IMPLEMENTED(rc != MCPU_ERR_UNSUPPORTED, what, ": ", msg);
  TORCH_CHECK(false, what, ": ", msg);
}

bool x_dtype(at::ScalarType s) {
  return s == at::kFloat || s == at::kBFloat16 || s == at::kHalf;
}

int32_t dtype_tag(at::ScalarType s) {
  return s == at::kFloat ? MCPU_F32 : (s == at::kBFloat16 ? MCPU_BF16 : MCPU_F16);
}

bool has(const optional<Tensor>& t) { return t.has_value() && t->defined(); }
const void* ptr(const optional<Tensor>& t) { return has(t) ? t->data_ptr() : nullptr; }
const float* fptr(const optional<Tensor>& t) {
  return has(t) ? static_cast<const float*>(t->data_ptr()) : nullptr;
}

void strides3(int64_t (&s)[3], const Tensor& t) {
  for (int i = 0; i < 3; ++i) s[i] = t.stride(i);
}
void strides3(int64_t (&s)[3], const optional<Tensor>& t) {
  if (has(t)) strides3(s, *t);
  else s[0] = s[1] = s[2] = 0;
}

void check_gpu(const char* name, const optional<Tensor>& t) {
  if (has(t))
    TORCH_CHECK_VALUE(t->is_cuda(), name, " runs on ROCm GPU tensors, got a tensor on ", t->device());
}

optional<Tensor> opt(const Tensor& t) { return t.defined() ? optional<Tensor>(t) : std::nullopt; }

// A (batch, dim, seqlen) result laid out like x: channel-contiguous when x is
// (the transposed views Hugging Face passes), contiguous otherwise.
Tensor like_x(const Tensor& x) {
  if (x.dim() == 3 && x.stride(1) == 1 && x.stride(2) != 1) {
    const int64_t b = x.size(0), d = x.size(1), l = x.size(2);
    return at::empty_strided({b, d, l}, {d * l, 1, d}, x.options());
  }
  return at::empty(x.sizes(), x.options());
}

// Float32 copy of a parameter tensor when it is not already float32 and
// contiguous (the reference computes in float32 whatever they are stored in).
Tensor f32c(const Tensor& t) { return t.scalar_type() == at::kFloat && t.is_contiguous() ? t : t.to(at::kFloat).contiguous(); }
optional<Tensor> f32c(const optional<Tensor>& t) { return has(t) ? optional<Tensor>(f32c(*t)) : std::nullopt; }

// ---- selective scan -------------------------------------------------------------

void validate_scan(const char* name, const Tensor& u, const Tensor& delta, const Tensor& A,
                   const Tensor& B, const Tensor& C, const optional<Tensor>& D,
                   const optional<Tensor>& z, const optional<Tensor>& bias,
                   std::initializer_list<optional<Tensor>> extra = {}) {
  for (const optional<Tensor>& t : {opt(u), opt(delta), opt(A), opt(B), opt(C), D, z, bias})
    check_gpu(name, t);
  for (const optional<Tensor>& t : extra) check_gpu(name, t);
  TORCH_CHECK_VALUE(x_dtype(u.scalar_type()) && delta.scalar_type() == u.scalar_type() &&
                        (!has(z) || z->scalar_type() == u.scalar_type()),
                    name, " expects u, delta and z of one dtype among float32, bfloat16 and float16");
  for (const optional<Tensor>& t : {opt(A), opt(B), opt(C), D, bias})
    TORCH_CHECK_VALUE(!has(t) || t->scalar_type() == at::kFloat, name,
                      " expects float32 A, B, C, D and delta_bias");
  TORCH_CHECK_VALUE(u.dim() == 3 && delta.sizes() == u.sizes() && (!has(z) || z->sizes() == u.sizes()),
                    name, " expects u, delta and z of shape (batch, dim, seqlen)");
  const int64_t batch = u.size(0), dim = u.size(1), seqlen = u.size(2);
  TORCH_CHECK_VALUE(A.dim() == 2 && A.size(0) == dim, name, " expects A of shape (dim, dstate)");
  const int64_t dstate = A.size(1);
  for (const Tensor* X : {&B, &C})
    TORCH_CHECK_VALUE(X->dim() == 4 && X->size(0) == batch && X->size(2) == seqlen &&
                          X->size(3) == dstate,
                      name, " expects B and C of shape (batch, ngroups, seqlen, dstate)");
  TORCH_CHECK_VALUE(B.size(1) == C.size(1) && B.size(1) > 0 && dim % B.size(1) == 0, name,
                    ": dim (", dim, ") must be divisible by ngroups (", B.size(1), ")");
  for (const optional<Tensor>& t : {D, bias})
    TORCH_CHECK_VALUE(!has(t) || (t->dim() == 1 && t->size(0) == dim && t->is_contiguous()), name,
                      " expects contiguous D and delta_bias of shape (dim,)");
  TORCH_CHECK_VALUE(A.is_contiguous(), name, " expects a contiguous A");
}

mcpu_scan_args scan_args(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
                         const Tensor& C, const optional<Tensor>& D, const optional<Tensor>& z,
                         const optional<Tensor>& bias, bool softplus) {
  mcpu_scan_args a;
  std::memset(&a, 0, sizeof(a));
  a.u = u.data_ptr();
  a.delta = delta.data_ptr();
  a.A = static_cast<const float*>(A.data_ptr());
  a.B = static_cast<const float*>(B.data_ptr());
  a.C = static_cast<const float*>(C.data_ptr());
  a.D = fptr(D);
  a.z = ptr(z);
  a.delta_bias = fptr(bias);
  a.batch = u.size(0);
  a.dim = u.size(1);
  a.seqlen = u.size(2);
  a.dstate = A.size(1);
  a.ngroups = B.size(1);
  a.delta_softplus = softplus ? 1 : 0;
  a.dtype = dtype_tag(u.scalar_type());
  strides3(a.u_stride, u);
  strides3(a.delta_stride, delta);
  strides3(a.z_stride, z);
  for (int i = 0; i < 4; ++i) {
    a.B_stride[i] = B.stride(i);
    a.C_stride[i] = C.stride(i);
  }
  return a;
}

constexpr int64_t kBlockT = 16;  // time steps per checkpoint block

std::vector<int64_t> ckpt_shape(const Tensor& u, const Tensor& A) {
  return {u.size(0), u.size(1), (u.size(2) + kBlockT - 1) / kBlockT, A.size(1)};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> scan_fwd_impl(
    const char* name, const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
    const Tensor& C, const optional<Tensor>& D, const optional<Tensor>& z,
    const optional<Tensor>& bias, bool softplus, bool save) {
  validate_scan(name, u, delta, A, B, C, D, z, bias);
  c10::DeviceGuard guard(u.device());
  const int64_t batch = u.size(0), dim = u.size(1);
  Tensor out = like_x(u);
  Tensor last = at::empty({batch, dim, A.size(1)}, u.options().dtype(at::kFloat));
  Tensor ckpt, ysave;
  mcpu_scan_args a = scan_args(u, delta, A, B, C, D, z, bias, softplus);
  a.out = out.data_ptr();
  strides3(a.out_stride, out);
  a.last_state = static_cast<float*>(last.data_ptr());
  if (save) {
    ckpt = at::empty(ckpt_shape(u, A), u.options().dtype(at::kFloat));
    ysave = has(z) ? at::empty(u.sizes(), u.options()) : at::empty({0}, u.options());
    a.ckpt = static_cast<float*>(ckpt.data_ptr());
    a.ysave = has(z) ? ysave.data_ptr() : nullptr;
  }
  const size_t ws_bytes = mcpu_selective_scan_fwd_workspace_size(&a);
  Tensor ws;
  if (ws_bytes > 0) ws = at::empty({static_cast<int64_t>(ws_bytes)}, u.options().dtype(at::kByte));
  check_rc(mcpu_selective_scan_fwd(&a, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
                                   stream_of(u)),
           name);
  return {out, last, ckpt, ysave};
}

std::tuple<Tensor, Tensor> selective_scan_fwd(const Tensor& u, const Tensor& delta, const Tensor& A,
                                              const Tensor& B, const Tensor& C,
                                              const optional<Tensor>& D, const optional<Tensor>& z,
                                              const optional<Tensor>& bias, bool softplus) {
  auto r = scan_fwd_impl("mamba_cpu::selective_scan_fwd", u, delta, A, B, C, D, z, bias, softplus,
                         false);
  return {std::get<0>(r), std::get<1>(r)};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> selective_scan_fwd_ckpt(
    const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B, const Tensor& C,
    const optional<Tensor>& D, const optional<Tensor>& z, const optional<Tensor>& bias,
    bool softplus) {
  return scan_fwd_impl("mamba_cpu::selective_scan_fwd_ckpt", u, delta, A, B, C, D, z, bias,
                       softplus, true);
}

using Grads8 = std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>;

// dz_into: an existing (batch, dim, seqlen) view to write dz into (any
// strides), instead of a new tensor.
Grads8 scan_bwd_impl(const char* name, const Tensor& u, const Tensor& delta, const Tensor& A,
                     const Tensor& B, const Tensor& C, const optional<Tensor>& D,
                     const optional<Tensor>& z, const optional<Tensor>& bias, bool softplus,
                     const Tensor& dout, const optional<Tensor>& dlast_state,
                     const optional<Tensor>& ckpt, const optional<Tensor>& ysave_in,
                     const Tensor* dz_into = nullptr) {
  validate_scan(name, u, delta, A, B, C, D, z, bias, {opt(dout), dlast_state, ckpt, ysave_in});
  TORCH_CHECK_VALUE(dout.sizes() == u.sizes() && dout.scalar_type() == u.scalar_type(), name,
                    " expects dout shaped and typed like u");
  const int64_t batch = u.size(0), dim = u.size(1), dstate = A.size(1);
  optional<Tensor> dlast;
  if (has(dlast_state)) {
    TORCH_CHECK_VALUE(dlast_state->scalar_type() == at::kFloat && dlast_state->dim() == 3 &&
                          dlast_state->size(0) == batch && dlast_state->size(1) == dim &&
                          dlast_state->size(2) == dstate,
                      name, " expects float32 dlast_state (batch, dim, dstate)");
    dlast = dlast_state->contiguous();
  }
  if (has(ckpt))
    TORCH_CHECK_VALUE(ckpt->scalar_type() == at::kFloat && ckpt->is_contiguous() &&
                          ckpt->sizes() == at::IntArrayRef(ckpt_shape(u, A)),
                      name, " expects the float32 checkpoints written by selective_scan_fwd_ckpt");
  optional<Tensor> ysave = (has(ysave_in) && ysave_in->numel() > 0) ? ysave_in : std::nullopt;
  if (has(ysave))
    TORCH_CHECK_VALUE(ysave->sizes() == u.sizes() && ysave->scalar_type() == u.scalar_type() &&
                          ysave->is_contiguous() && has(z),
                      name, " expects the y written by selective_scan_fwd_ckpt");
  c10::DeviceGuard guard(u.device());
  // Gradients take their input's layout (channel-contiguous stays so).
  Tensor du = like_x(u);
  Tensor ddelta = like_x(delta);
  Tensor dA = at::empty(A.sizes(), A.options());
  Tensor dB = at::empty(B.sizes(), B.options());
  Tensor dC = at::empty(C.sizes(), C.options());
  Tensor dD = at::empty({dim}, A.options());
  Tensor dz = has(z) ? (dz_into != nullptr ? *dz_into : like_x(*z)) : at::empty({0}, u.options());
  Tensor dbias = at::empty({dim}, A.options());
  mcpu_scan_args a = scan_args(u, delta, A, B, C, D, z, bias, softplus);
  a.dout = dout.data_ptr();
  strides3(a.dout_stride, dout);
  a.dlast_state = fptr(dlast);
  a.ckpt = has(ckpt) ? static_cast<float*>(ckpt->data_ptr()) : nullptr;
  a.ysave = has(ysave) ? ysave->data_ptr() : nullptr;
  a.du = du.data_ptr();
  a.ddelta = ddelta.data_ptr();
  a.dz = has(z) ? dz.data_ptr() : nullptr;
  strides3(a.du_stride, du);
  strides3(a.ddelta_stride, ddelta);
  if (has(z)) strides3(a.dz_stride, dz);
  a.dA = static_cast<float*>(dA.data_ptr());
  a.dB = static_cast<float*>(dB.data_ptr());
  a.dC = static_cast<float*>(dC.data_ptr());
  a.dD = static_cast<float*>(dD.data_ptr());
  a.ddelta_bias = static_cast<float*>(dbias.data_ptr());
  const size_t ws_bytes = mcpu_selective_scan_bwd_workspace_size(&a);
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)},
                        u.options().dtype(at::kByte));
  check_rc(mcpu_selective_scan_bwd(&a, ws.data_ptr(), ws_bytes, stream_of(u)), name);
  return {du, ddelta, dA, dB, dC, dD, dz, dbias};
}

Grads8 selective_scan_bwd(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
                          const Tensor& C, const optional<Tensor>& D, const optional<Tensor>& z,
                          const optional<Tensor>& bias, bool softplus, const Tensor& dout,
                          const optional<Tensor>& dlast_state) {
  return scan_bwd_impl("mamba_cpu::selective_scan_bwd", u, delta, A, B, C, D, z, bias, softplus,
                       dout, dlast_state, std::nullopt, std::nullopt);
}

Grads8 selective_scan_bwd_ckpt(const Tensor& u, const Tensor& delta, const Tensor& A,
                               const Tensor& B, const Tensor& C, const optional<Tensor>& D,
                               const optional<Tensor>& z, const optional<Tensor>& bias,
                               bool softplus, const Tensor& dout,
                               const optional<Tensor>& dlast_state, const Tensor& ckpt,
                               const Tensor& ysave) {
  return scan_bwd_impl("mamba_cpu::selective_scan_bwd_ckpt", u, delta, A, B, C, D, z, bias,
                       softplus, dout, dlast_state, ckpt, ysave);
}

// Autograd (reference selective_scan_interface.py:100-124): inputs are saved,
// never activations; a missing output gradient is zero; gradients of absent
// D / z / delta_bias are None.
template <bool CKPT>
struct ScanFn : public torch::autograd::Function<ScanFn<CKPT>> {
  static variable_list forward(AutogradContext* ctx, const Tensor& u, const Tensor& delta,
                               const Tensor& A, const Tensor& B, const Tensor& C,
                               const optional<Tensor>& D, const optional<Tensor>& z,
                               const optional<Tensor>& bias, bool softplus) {
    at::AutoDispatchBelowADInplaceOrView below;
    variable_list out;
    Tensor ckpt, ysave;
    if constexpr (CKPT) {
      static auto op = c10::Dispatcher::singleton()
                           .findSchemaOrThrow("mamba_cpu::selective_scan_fwd_ckpt", "")
                           .typed<decltype(selective_scan_fwd_ckpt)>();
      auto r = op.call(u, delta, A, B, C, D, z, bias, softplus);
      ckpt = std::get<2>(r);
      ysave = std::get<3>(r);
      out = {std::get<0>(r), std::get<1>(r), ckpt, ysave};
      ctx->mark_non_differentiable({ckpt, ysave});
    } else {
      static auto op = c10::Dispatcher::singleton()
                           .findSchemaOrThrow("mamba_cpu::selective_scan_fwd", "")
                           .typed<decltype(selective_scan_fwd)>();
      auto r = op.call(u, delta, A, B, C, D, z, bias, softplus);
      out = {std::get<0>(r), std::get<1>(r)};
    }
    ctx->save_for_backward({u, delta, A, B, C, D.value_or(Tensor()), z.value_or(Tensor()),
                            bias.value_or(Tensor()), ckpt, ysave});
    ctx->saved_data["softplus"] = softplus;
    ctx->set_materialize_grads(false);
    return out;
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const variable_list s = ctx->get_saved_variables();
    const Tensor &u = s[0], &delta = s[1], &A = s[2], &B = s[3], &C = s[4];
    const optional<Tensor> D = opt(s[5]), z = opt(s[6]), bias = opt(s[7]);
    const bool softplus = ctx->saved_data["softplus"].toBool();
    const Tensor dout = grads[0].defined() ? grads[0].to(u.scalar_type()) : at::zeros_like(u);
    const optional<Tensor> dlast =
        grads[1].defined() ? optional<Tensor>(grads[1].to(at::kFloat).contiguous()) : std::nullopt;
    Grads8 g;
    if constexpr (CKPT) {
      static auto op = c10::Dispatcher::singleton()
                           .findSchemaOrThrow("mamba_cpu::selective_scan_bwd_ckpt", "")
                           .typed<decltype(selective_scan_bwd_ckpt)>();
      g = op.call(u, delta, A, B, C, D, z, bias, softplus, dout, dlast, s[8], s[9]);
    } else {
      static auto op = c10::Dispatcher::singleton()
                           .findSchemaOrThrow("mamba_cpu::selective_scan_bwd", "")
                           .typed<decltype(selective_scan_bwd)>();
      g = op.call(u, delta, A, B, C, D, z, bias, softplus, dout, dlast);
    }
    return {std::get<0>(g), std::get<1>(g), std::get<2>(g), std::get<3>(g), std::get<4>(g),
            has(D) ? std::get<5>(g) : Tensor(), has(z) ? std::get<6>(g) : Tensor(),
            has(bias) ? std::get<7>(g) : Tensor(), Tensor()};
  }
};

std::tuple<Tensor, Tensor> selective_scan_fwd_autograd(
    const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B, const Tensor& C,
    const optional<Tensor>& D, const optional<Tensor>& z, const optional<Tensor>& bias,
    bool softplus) {
  auto r = ScanFn<false>::apply(u, delta, A, B, C, D, z, bias, softplus);
  return {r[0], r[1]};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> selective_scan_fwd_ckpt_autograd(
    const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B, const Tensor& C,
    const optional<Tensor>& D, const optional<Tensor>& z, const optional<Tensor>& bias,
    bool softplus) {
  auto r = ScanFn<true>::apply(u, delta, A, B, C, D, z, bias, softplus);
  return {r[0], r[1], r[2], r[3]};
}

// ---- selective scan, complex A ------------------------------------------------------
//
// mamba_ssm's complex-A scan (the reference rejects complex A,
// selective_scan_interface.py:160-161). A is complex64 (dim, dstate); B and C
// reach the operators as float32 (batch, ngroups, seqlen, dstate, 2) views
// whose last dim is the (re, im) pair (unit stride), so both mamba_ssm's real
// (batch, ngroups, dstate, 2 seqlen) layout and a complex tensor's
// view_as_real pass without copies. The forward also returns the block
// checkpoints its backward restarts from; autograd is wired in Python.

void validate_cscan(const char* name, const Tensor& u, const Tensor& delta, const Tensor& A,
                    const Tensor& B, const Tensor& C, const optional<Tensor>& D,
                    const optional<Tensor>& z, const optional<Tensor>& bias,
                    std::initializer_list<optional<Tensor>> extra = {}) {
  for (const optional<Tensor>& t : {opt(u), opt(delta), opt(A), opt(B), opt(C), D, z, bias})
    check_gpu(name, t);
  for (const optional<Tensor>& t : extra) check_gpu(name, t);
  TORCH_CHECK_VALUE(x_dtype(u.scalar_type()) && delta.scalar_type() == u.scalar_type() &&
                        (!has(z) || z->scalar_type() == u.scalar_type()),
                    name, " expects u, delta and z of one dtype among float32, bfloat16 and float16");
  TORCH_CHECK_VALUE(u.dim() == 3 && delta.sizes() == u.sizes() && (!has(z) || z->sizes() == u.sizes()),
                    name, " expects u, delta and z of shape (batch, dim, seqlen)");
  const int64_t batch = u.size(0), dim = u.size(1), seqlen = u.size(2);
  TORCH_CHECK_VALUE(A.scalar_type() == at::kComplexFloat && A.dim() == 2 && A.size(0) == dim &&
                        A.is_contiguous(),
                    name, " expects a contiguous complex64 A of shape (dim, dstate)");
  const int64_t dstate = A.size(1);
  for (const Tensor* X : {&B, &C})
    TORCH_CHECK_VALUE(X->scalar_type() == at::kFloat && X->dim() == 5 && X->size(0) == batch &&
                          X->size(2) == seqlen && X->size(3) == dstate && X->size(4) == 2 &&
                          X->stride(4) == 1,
                      name, " expects float32 B and C of shape (batch, ngroups, seqlen, dstate, 2) "
                      "with (re, im) pairs in the unit-stride last dim");
  TORCH_CHECK_VALUE(B.size(1) == C.size(1) && B.size(1) > 0 && dim % B.size(1) == 0, name,
                    ": dim (", dim, ") must be divisible by ngroups (", B.size(1), ")");
  for (const optional<Tensor>& t : {D, bias})
    TORCH_CHECK_VALUE(!has(t) || (t->scalar_type() == at::kFloat && t->dim() == 1 &&
                                  t->size(0) == dim && t->is_contiguous()),
                      name, " expects contiguous float32 D and delta_bias of shape (dim,)");
}

mcpu_scan_args cscan_args(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
                          const Tensor& C, const optional<Tensor>& D, const optional<Tensor>& z,
                          const optional<Tensor>& bias, bool softplus) {
  mcpu_scan_args a;
  std::memset(&a, 0, sizeof(a));
  a.complex_a = 1;
  a.u = u.data_ptr();
  a.delta = delta.data_ptr();
  a.A = static_cast<const float*>(A.data_ptr());
  a.B = static_cast<const float*>(B.data_ptr());
  a.C = static_cast<const float*>(C.data_ptr());
  a.D = fptr(D);
  a.z = ptr(z);
  a.delta_bias = fptr(bias);
  a.batch = u.size(0);
  a.dim = u.size(1);
  a.seqlen = u.size(2);
  a.dstate = A.size(1);
  a.ngroups = B.size(1);
  a.delta_softplus = softplus ? 1 : 0;
  a.dtype = dtype_tag(u.scalar_type());
  strides3(a.u_stride, u);
  strides3(a.delta_stride, delta);
  strides3(a.z_stride, z);
  for (int i = 0; i < 4; ++i) {
    a.B_stride[i] = B.stride(i);
    a.C_stride[i] = C.stride(i);
  }
  return a;
}

std::vector<int64_t> cckpt_shape(const Tensor& u, const Tensor& A) {
  return {u.size(0), u.size(1), (u.size(2) + kBlockT - 1) / kBlockT, A.size(1), 2};
}

std::tuple<Tensor, Tensor, Tensor> selective_scan_cfwd(const Tensor& u, const Tensor& delta,
                                                       const Tensor& A, const Tensor& B,
                                                       const Tensor& C, const optional<Tensor>& D,
                                                       const optional<Tensor>& z,
                                                       const optional<Tensor>& bias, bool softplus) {
  const char* name = "mamba_cpu::selective_scan_cfwd";
  validate_cscan(name, u, delta, A, B, C, D, z, bias);
  c10::DeviceGuard guard(u.device());
  Tensor out = like_x(u);
  Tensor last = at::empty({u.size(0), u.size(1), A.size(1)}, u.options().dtype(at::kComplexFloat));
  Tensor ckpt = at::empty(cckpt_shape(u, A), u.options().dtype(at::kFloat));
  mcpu_scan_args a = cscan_args(u, delta, A, B, C, D, z, bias, softplus);
  a.out = out.data_ptr();
  strides3(a.out_stride, out);
  a.last_state = static_cast<float*>(last.data_ptr());
  a.ckpt = static_cast<float*>(ckpt.data_ptr());
  // Above 32 states the slices' shares of y need a workspace.
  const size_t ws_bytes = mcpu_selective_scan_fwd_workspace_size(&a);
  Tensor ws;
  if (ws_bytes > 0) ws = at::empty({static_cast<int64_t>(ws_bytes)}, u.options().dtype(at::kByte));
  check_rc(mcpu_selective_scan_fwd(&a, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream_of(u)), name);
  return {out, last, ckpt};
}

Grads8 selective_scan_cbwd(const Tensor& u, const Tensor& delta, const Tensor& A, const Tensor& B,
                           const Tensor& C, const optional<Tensor>& D, const optional<Tensor>& z,
                           const optional<Tensor>& bias, bool softplus, const Tensor& dout,
                           const optional<Tensor>& dlast_state, const optional<Tensor>& ckpt) {
  const char* name = "mamba_cpu::selective_scan_cbwd";
  validate_cscan(name, u, delta, A, B, C, D, z, bias, {opt(dout), dlast_state, ckpt});
  TORCH_CHECK_VALUE(dout.sizes() == u.sizes() && dout.scalar_type() == u.scalar_type(), name,
                    " expects dout shaped and typed like u");
  const int64_t batch = u.size(0), dim = u.size(1), dstate = A.size(1);
  optional<Tensor> dlast;
  if (has(dlast_state)) {
    TORCH_CHECK_VALUE(dlast_state->scalar_type() == at::kComplexFloat && dlast_state->dim() == 3 &&
                          dlast_state->size(0) == batch && dlast_state->size(1) == dim &&
                          dlast_state->size(2) == dstate,
                      name, " expects complex64 dlast_state (batch, dim, dstate)");
    dlast = dlast_state->contiguous();
  }
  if (has(ckpt))
    TORCH_CHECK_VALUE(ckpt->scalar_type() == at::kFloat && ckpt->is_contiguous() &&
                          ckpt->sizes() == at::IntArrayRef(cckpt_shape(u, A)),
                      name, " expects the checkpoints written by selective_scan_cfwd");
  c10::DeviceGuard guard(u.device());
  Tensor du = like_x(u);
  Tensor ddelta = like_x(delta);
  Tensor dA = at::empty(A.sizes(), A.options());
  Tensor dB = at::empty(B.sizes(), B.options());
  Tensor dC = at::empty(C.sizes(), C.options());
  Tensor dD = at::empty({dim}, B.options());
  Tensor dz = has(z) ? like_x(*z) : at::empty({0}, u.options());
  Tensor dbias = at::empty({dim}, B.options());
  mcpu_scan_args a = cscan_args(u, delta, A, B, C, D, z, bias, softplus);
  a.dout = dout.data_ptr();
  strides3(a.dout_stride, dout);
  a.dlast_state = has(dlast) ? static_cast<const float*>(dlast->data_ptr()) : nullptr;
  a.ckpt = has(ckpt) ? static_cast<float*>(ckpt->data_ptr()) : nullptr;
  a.du = du.data_ptr();
  a.ddelta = ddelta.data_ptr();
  a.dz = has(z) ? dz.data_ptr() : nullptr;
  strides3(a.du_stride, du);
  strides3(a.ddelta_stride, ddelta);
  if (has(z)) strides3(a.dz_stride, dz);
  a.dA = static_cast<float*>(dA.data_ptr());
  a.dB = static_cast<float*>(dB.data_ptr());
  a.dC = static_cast<float*>(dC.data_ptr());
  a.dD = static_cast<float*>(dD.data_ptr());
  a.ddelta_bias = static_cast<float*>(dbias.data_ptr());
  const size_t ws_bytes = mcpu_selective_scan_bwd_workspace_size(&a);
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)},
                        u.options().dtype(at::kByte));
  check_rc(mcpu_selective_scan_bwd(&a, ws.data_ptr(), ws_bytes, stream_of(u)), name);
  return {du, ddelta, dA, dB, dC, dD, dz, dbias};
}

// ---- causal conv1d ------------------------------------------------------------------

void check_conv(const char* name, const Tensor& x, const Tensor& weight,
                const optional<Tensor>& bias, const optional<Tensor>& init) {
  for (const optional<Tensor>& t : {opt(x), opt(weight), bias, init}) check_gpu(name, t);
  TORCH_CHECK_VALUE(x_dtype(x.scalar_type()), name,
                    " expects x in float32, bfloat16 or float16, got ", x.scalar_type());
  TORCH_CHECK_VALUE(x.dim() == 3 && weight.dim() == 2 && weight.size(0) == x.size(1), name,
                    " expects x (batch, dim, seqlen) and weight (dim, width)");
  TORCH_CHECK_VALUE(weight.scalar_type() == at::kFloat && weight.is_contiguous(), name,
                    " expects a contiguous float32 weight");
  TORCH_CHECK_VALUE(!has(bias) || (bias->scalar_type() == at::kFloat && bias->dim() == 1 &&
                                   bias->size(0) == x.size(1)),
                    name, " expects a float32 bias of shape (dim,)");
  TORCH_CHECK_VALUE(!has(init) || (init->scalar_type() == x.scalar_type() && init->dim() == 3 &&
                                   init->size(0) == x.size(0) && init->size(1) == x.size(1) &&
                                   init->size(2) == weight.size(1) - 1),
                    name, " expects initial_states (batch, dim, width - 1) in x's dtype");
}

// Optional (batch, seqlen) packed-sequence ids of the conv.
void check_seq_idx(const char* name, const optional<Tensor>& seq_idx, const Tensor& x) {
  if (!has(seq_idx)) return;
  check_gpu(name, seq_idx);
  TORCH_CHECK_VALUE(seq_idx->scalar_type() == at::kInt && seq_idx->dim() == 2 &&
                        seq_idx->size(0) == x.size(0) && seq_idx->size(1) == x.size(2) &&
                        seq_idx->is_contiguous(),
                    name, " expects seq_idx as a contiguous int32 tensor of shape (batch, seqlen)");
}

mcpu_conv_args conv_args(const Tensor& x, const Tensor& weight, const optional<Tensor>& bias,
                         const optional<Tensor>& init, bool silu,
                         const optional<Tensor>& seq_idx = std::nullopt) {
  mcpu_conv_args a;
  std::memset(&a, 0, sizeof(a));
  a.seq_idx = has(seq_idx) ? static_cast<const int32_t*>(seq_idx->data_ptr()) : nullptr;
  a.x = x.data_ptr();
  a.weight = static_cast<const float*>(weight.data_ptr());
  a.bias = fptr(bias);
  a.initial_states = ptr(init);
  a.batch = x.size(0);
  a.dim = x.size(1);
  a.seqlen = x.size(2);
  a.width = weight.size(1);
  a.silu = silu ? 1 : 0;
  a.dtype = dtype_tag(x.scalar_type());
  strides3(a.x_stride, x);
  strides3(a.init_stride, init);
  return a;
}

std::tuple<Tensor, Tensor> causal_conv1d_fwd(const Tensor& x, const Tensor& weight,
                                             const optional<Tensor>& bias,
                                             const optional<Tensor>& init,
                                             bool return_final_states, bool silu,
                                             const optional<Tensor>& seq_idx) {
  const char* name = "mamba_cpu::causal_conv1d_fwd";
  check_conv(name, x, weight, bias, init);
  c10::DeviceGuard guard(x.device());
  Tensor out = like_x(x);
  const int64_t b = x.size(0), d = x.size(1), w = weight.size(1);
  Tensor final = return_final_states ? at::empty({b, d, w - 1}, x.options())
                                     : at::empty({0}, x.options());
  check_seq_idx("mamba_cpu::causal_conv1d_fwd", seq_idx, x);
  mcpu_conv_args a = conv_args(x, weight, bias, init, silu, seq_idx);
  a.out = out.data_ptr();
  strides3(a.out_stride, out);
  a.final_states = return_final_states ? final.data_ptr() : nullptr;
  check_rc(mcpu_causal_conv1d_fwd(&a, stream_of(x)), name);
  return {out, final};
}

// dx_into: an existing (batch, dim, seqlen) view to write dx into (any
// strides), instead of a new tensor.
std::tuple<Tensor, Tensor, Tensor, Tensor> conv_bwd_impl(
    const Tensor& x, const Tensor& weight, const optional<Tensor>& bias,
    const optional<Tensor>& init, const Tensor& dout, const optional<Tensor>& dfinal_states,
    bool silu, const optional<Tensor>& seq_idx, const Tensor* dx_into) {
  const char* name = "mamba_cpu::causal_conv1d_bwd";
  check_seq_idx(name, seq_idx, x);
  check_conv(name, x, weight, bias, init);
  check_gpu(name, dout);
  check_gpu(name, dfinal_states);
  TORCH_CHECK_VALUE(dout.sizes() == x.sizes() && dout.scalar_type() == x.scalar_type(), name,
                    " expects dout shaped and typed like x");
  const int64_t b = x.size(0), d = x.size(1), w = weight.size(1);
  optional<Tensor> dfinal;
  if (has(dfinal_states)) {
    TORCH_CHECK_VALUE(dfinal_states->dim() == 3 && dfinal_states->size(0) == b &&
                          dfinal_states->size(1) == d && dfinal_states->size(2) == w - 1,
                      name, " expects dfinal_states (batch, dim, width - 1)");
    dfinal = dfinal_states->to(x.scalar_type()).contiguous();
  }
  c10::DeviceGuard guard(x.device());
  Tensor dx = dx_into != nullptr ? *dx_into : like_x(x);
  Tensor dweight = at::empty(weight.sizes(), weight.options());
  Tensor dbias = has(bias) ? at::empty({d}, weight.options()) : at::empty({0}, weight.options());
  Tensor dinit = has(init) ? at::empty({b, d, w - 1}, x.options()) : at::empty({0}, x.options());
  mcpu_conv_args a = conv_args(x, weight, bias, init, silu, seq_idx);
  a.dout = dout.data_ptr();
  strides3(a.dout_stride, dout);
  a.dfinal_states = ptr(dfinal);
  a.dx = dx.data_ptr();
  strides3(a.dx_stride, dx);
  a.dweight = static_cast<float*>(dweight.data_ptr());
  a.dbias = has(bias) ? static_cast<float*>(dbias.data_ptr()) : nullptr;
  a.dinitial_states = has(init) ? dinit.data_ptr() : nullptr;
  const size_t ws_bytes = mcpu_causal_conv1d_bwd_workspace_size(&a);
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes > 0 ? ws_bytes : 1)},
                        x.options().dtype(at::kByte));
  check_rc(mcpu_causal_conv1d_bwd(&a, ws.data_ptr(), ws_bytes, stream_of(x)), name);
  return {dx, dweight, dbias, dinit};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> causal_conv1d_bwd(
    const Tensor& x, const Tensor& weight, const optional<Tensor>& bias,
    const optional<Tensor>& init, const Tensor& dout, const optional<Tensor>& dfinal_states,
    bool silu, const optional<Tensor>& seq_idx) {
  return conv_bwd_impl(x, weight, bias, init, dout, dfinal_states, silu, seq_idx, nullptr);
}

struct ConvFn : public torch::autograd::Function<ConvFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& x, const Tensor& weight,
                               const optional<Tensor>& bias, const optional<Tensor>& init,
                               bool return_final_states, bool silu,
                               const optional<Tensor>& seq_idx) {
    at::AutoDispatchBelowADInplaceOrView below;
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("mamba_cpu::causal_conv1d_fwd", "")
                         .typed<decltype(causal_conv1d_fwd)>();
    auto r = op.call(x, weight, bias, init, return_final_states, silu, seq_idx);
    ctx->save_for_backward({x, weight, bias.value_or(Tensor()), init.value_or(Tensor()),
                            seq_idx.value_or(Tensor())});
    ctx->saved_data["silu"] = silu;
    ctx->saved_data["final"] = return_final_states;
    ctx->set_materialize_grads(false);
    return {std::get<0>(r), std::get<1>(r)};
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const variable_list s = ctx->get_saved_variables();
    const Tensor &x = s[0], &weight = s[1];
    const optional<Tensor> bias = opt(s[2]), init = opt(s[3]), seq_idx = opt(s[4]);
    const Tensor dout = grads[0].defined() ? grads[0].to(x.scalar_type()) : at::zeros_like(x);
    const optional<Tensor> dfinal = (ctx->saved_data["final"].toBool() && grads[1].defined())
                                        ? optional<Tensor>(grads[1])
                                        : std::nullopt;
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("mamba_cpu::causal_conv1d_bwd", "")
                         .typed<decltype(causal_conv1d_bwd)>();
    auto g = op.call(x, weight, bias, init, dout, dfinal, ctx->saved_data["silu"].toBool(), seq_idx);
    return {std::get<0>(g), std::get<1>(g), has(bias) ? std::get<2>(g) : Tensor(),
            has(init) ? std::get<3>(g) : Tensor(), Tensor(), Tensor(), Tensor()};
  }
};

std::tuple<Tensor, Tensor> causal_conv1d_fwd_autograd(const Tensor& x, const Tensor& weight,
                                                      const optional<Tensor>& bias,
                                                      const optional<Tensor>& init,
                                                      bool return_final_states, bool silu,
                                                      const optional<Tensor>& seq_idx) {
  auto r = ConvFn::apply(x, weight, bias, init, return_final_states, silu, seq_idx);
  return {r[0], r[1]};
}

// An optional (batch,) int32 index / length vector of the decode ops.
void check_index(const char* name, const char* what, const optional<Tensor>& t, int64_t batch) {
  if (!has(t)) return;
  check_gpu(name, t);
  TORCH_CHECK_VALUE(t->scalar_type() == at::kInt && t->dim() == 1 && t->size(0) == batch &&
                        t->is_contiguous(),
                    name, " expects ", what, " as a contiguous int32 tensor of shape (batch,)");
}

// Decode step(s) of the conv (ops/causal_conv1d.py:56-85): x (b, dim) for one
// step or (b, dim, seqlen); the output is shaped like x.
Tensor causal_conv1d_update(const Tensor& x, Tensor& conv_state, const Tensor& weight_in,
                            const optional<Tensor>& bias_in, bool silu,
                            const optional<Tensor>& cache_seqlens,
                            const optional<Tensor>& conv_state_indices) {
  const char* name = "mamba_cpu::causal_conv1d_update";
  for (const optional<Tensor>& t : {opt(x), opt(conv_state), opt(weight_in), bias_in}) check_gpu(name, t);
  check_index(name, "cache_seqlens", cache_seqlens, x.size(0));
  check_index(name, "conv_state_indices", conv_state_indices, x.size(0));
  TORCH_CHECK_VALUE(x_dtype(x.scalar_type()) && conv_state.scalar_type() == x.scalar_type(), name,
                    " expects x and conv_state of one dtype among float32, bfloat16 and float16");
  const bool single = x.dim() == 2;
  TORCH_CHECK_VALUE(weight_in.dim() == 2 && x.dim() >= 2 && weight_in.size(0) == x.size(1), name,
                    " expects weight (dim, width) with dim = x.size(1)");
  TORCH_CHECK_VALUE(!has(bias_in) || (bias_in->dim() == 1 && bias_in->size(0) == x.size(1)), name,
                    " expects bias of shape (dim,)");
  TORCH_CHECK_VALUE((single || x.dim() == 3) && conv_state.dim() == 3, name,
                    " expects x (batch, dim[, seqlen]) and conv_state (batch, dim, state_len)");
  TORCH_CHECK_VALUE(conv_state.size(1) == x.size(1) &&
                        (has(conv_state_indices) || conv_state.size(0) == x.size(0)),
                    name, " expects conv_state (batch, dim, state_len), or (rows, dim, state_len) "
                    "with conv_state_indices");
  TORCH_CHECK_VALUE(!has(cache_seqlens) || conv_state.size(2) >= 1, name,
                    " expects a conv_state of at least one slot when cache_seqlens is given");
  const Tensor weight = f32c(weight_in);
  const optional<Tensor> bias = f32c(bias_in);
  c10::DeviceGuard guard(x.device());
  Tensor out = at::empty(x.sizes(), x.options());
  mcpu_conv_update_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x.data_ptr();
  a.conv_state = conv_state.data_ptr();
  a.weight = static_cast<const float*>(weight.data_ptr());
  a.bias = fptr(bias);
  a.out = out.data_ptr();
  a.batch = x.size(0);
  a.dim = x.size(1);
  a.seqlen = single ? 1 : x.size(2);
  a.width = weight.size(1);
  a.state_len = conv_state.size(2);
  a.silu = silu ? 1 : 0;
  a.dtype = dtype_tag(x.scalar_type());
  auto s3 = [&](int64_t (&d)[3], const Tensor& t) {
    d[0] = t.stride(0);
    d[1] = t.stride(1);
    d[2] = single ? 0 : t.stride(2);
  };
  s3(a.x_stride, x);
  strides3(a.state_stride, conv_state);
  s3(a.out_stride, out);
  a.cache_seqlens = has(cache_seqlens) ? static_cast<const int32_t*>(cache_seqlens->data_ptr()) : nullptr;
  a.conv_state_indices =
      has(conv_state_indices) ? static_cast<const int32_t*>(conv_state_indices->data_ptr()) : nullptr;
  a.state_batch = conv_state.size(0);
  check_rc(mcpu_causal_conv1d_update(&a, stream_of(x)), name);
  return out;
}

// ---- fused Mamba-1 mixer (mamba_inner_fn) --------------------------------------------
//
// The forward and backward of mamba_inner_fn (without the optional RMS norms)
// as two operators, so that a training step issues its conv, scan and GEMM
// calls from C++ instead of one Python call each. Everything between in_proj
// and out_proj stays in the (batch, seqlen, channels) layout of in_proj's
// output: xz is the transposed view transformers passes, the conv and scan
// read and write those views through their strides, and the backward writes
// dx and dz straight into the two halves of one (batch, seqlen, 2 dim)
// gradient.

// Plain float32 GEMMs of the mixer through rocBLAS: its host cost per call
// is about 7.5 us against about 19 us through torch's default hipBLASLt path
// (a mixer layer makes nine of them per training step, and at the Mamba-130M
// training shape the step is bound by host time). One handle per thread and
// device (rocBLAS handles are not shared across threads; the autograd engine
// runs backward on its own thread), created on first use and kept.
constexpr int kMaxBlasDevices = 64;

rocblas_handle blas_handle(const Tensor& t) {
  thread_local rocblas_handle handles[kMaxBlasDevices] = {};
  const int dev = t.device().index();
  TORCH_CHECK(dev >= 0 && dev < kMaxBlasDevices, "mamba_cpu: device index ", dev, " out of range");
  if (handles[dev] == nullptr)
    TORCH_CHECK(rocblas_create_handle(&handles[dev]) == rocblas_status_success,
                "mamba_cpu: rocblas_create_handle failed");
  TORCH_CHECK(rocblas_set_stream(handles[dev], static_cast<hipStream_t>(stream_of(t))) ==
                  rocblas_status_success, "mamba_cpu: rocblas_set_stream failed");
  return handles[dev];
}

// How rocBLAS (column-major) sees a 2-D view: a row-major (r, c) matrix with
// row stride ld is its transpose stored column-major with leading dim ld.
bool blas_view(const Tensor& x, rocblas_operation& op, int64_t& ld) {
  const int64_t r = x.size(0), c = x.size(1);
  if (x.stride(1) == 1 && x.stride(0) >= std::max<int64_t>(c, 1)) {
    op = rocblas_operation_none;
    ld = x.stride(0);
    return true;
  }
  if (x.stride(0) == 1 && x.stride(1) >= std::max<int64_t>(r, 1)) {
    op = rocblas_operation_transpose;
    ld = x.stride(1);
    return true;
  }
  return false;
}

// c = a @ b + beta * c for float32 2-D views a (m, k), b (k, n) and a
// row-major c (m, n) with unit column stride; a and b row- or column-major.
void gemm_into(const Tensor& a, const Tensor& b, const Tensor& c, float beta) {
  const int64_t m = a.size(0), k = a.size(1), n = b.size(1);
  TORCH_CHECK(b.size(0) == k && c.size(0) == m && c.size(1) == n && c.stride(1) == 1 &&
                  c.stride(0) >= std::max<int64_t>(n, 1),
              "mamba_cpu: gemm shapes");
  if (m == 0 || n == 0) return;
  if (k == 0) {
    if (beta == 0.f) c.zero_();
    else c.mul_(beta);
    return;
  }
  rocblas_operation opa, opb;
  int64_t lda, ldb;
  if (!blas_view(a, opa, lda)) return gemm_into(a.contiguous(), b, c, beta);
  if (!blas_view(b, opb, ldb)) return gemm_into(a, b.contiguous(), c, beta);
  const int64_t big = std::numeric_limits<rocblas_int>::max();
  TORCH_CHECK(m <= big && n <= big && k <= big && lda <= big && ldb <= big && c.stride(0) <= big,
              "mamba_cpu: gemm too large");
  const float alpha = 1.f;
  // Column-major: c^T (n, m) = b^T (n, k) a^T (k, m).
  TORCH_CHECK(rocblas_sgemm(blas_handle(c), opb, opa, static_cast<rocblas_int>(n), static_cast<rocblas_int>(m),
                            static_cast<rocblas_int>(k), &alpha, static_cast<const float*>(b.data_ptr()),
                            static_cast<rocblas_int>(ldb), static_cast<const float*>(a.data_ptr()),
                            static_cast<rocblas_int>(lda), &beta, static_cast<float*>(c.data_ptr()),
                            static_cast<rocblas_int>(c.stride(0))) == rocblas_status_success,
              "mamba_cpu: rocblas_sgemm failed");
}

Tensor gemm(const Tensor& a, const Tensor& b) {
  Tensor c = at::empty({a.size(0), b.size(1)}, a.options());
  gemm_into(a, b, c, 0.f);
  return c;
}

void check_inner(const char* name, const Tensor& xz, const Tensor& conv_w, const Tensor& x_proj_w,
                 const Tensor& dt_proj_w, const Tensor& out_proj_w, const Tensor& A) {
  for (const Tensor* t : {&xz, &conv_w, &x_proj_w, &dt_proj_w, &out_proj_w, &A}) {
    check_gpu(name, opt(*t));
    TORCH_CHECK_VALUE(t->scalar_type() == at::kFloat, name, " runs float32 tensors");
  }
  TORCH_CHECK_VALUE(xz.dim() == 3 && xz.size(1) % 2 == 0, name, " expects xz (batch, 2 dim, seqlen)");
  const int64_t d = xz.size(1) / 2;
  TORCH_CHECK_VALUE(A.dim() == 2 && A.size(0) == d, name, " expects A (dim, dstate)");
  const int64_t R = dt_proj_w.size(1), N = A.size(1);
  TORCH_CHECK_VALUE(conv_w.numel() % d == 0 && conv_w.size(0) == d, name, " expects conv1d_weight (dim, [1,] width)");
  TORCH_CHECK_VALUE(x_proj_w.dim() == 2 && x_proj_w.size(0) == R + 2 * N && x_proj_w.size(1) == d, name,
                    " expects x_proj_weight (dt_rank + 2 dstate, dim)");
  TORCH_CHECK_VALUE(dt_proj_w.dim() == 2 && dt_proj_w.size(0) == d, name, " expects delta_proj_weight (dim, dt_rank)");
  TORCH_CHECK_VALUE(out_proj_w.dim() == 2 && out_proj_w.size(1) == d, name, " expects out_proj_weight (d_model, dim)");
}

// Returns (out, conv_out, x_dbl, delta, ckpt, ysave, y): out (batch, seqlen,
// d_model) and what the backward restarts from.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> mamba_inner_fwd(
    const Tensor& xz, const Tensor& conv_w, const optional<Tensor>& conv_b, const Tensor& x_proj_w,
    const Tensor& dt_proj_w, const Tensor& out_proj_w, const optional<Tensor>& out_proj_b,
    const Tensor& A, const optional<Tensor>& D, const optional<Tensor>& delta_bias, bool softplus) {
  const char* name = "mamba_cpu::mamba_inner_fwd";
  check_inner(name, xz, conv_w, x_proj_w, dt_proj_w, out_proj_w, A);
  c10::DeviceGuard guard(xz.device());
  const int64_t d = xz.size(1) / 2, R = dt_proj_w.size(1), N = A.size(1);
  const Tensor x = xz.narrow(1, 0, d), z = xz.narrow(1, d, d);
  const Tensor w2 = conv_w.reshape({d, -1}).contiguous();
  const Tensor conv_out = std::get<0>(causal_conv1d_fwd(x, w2, f32c(conv_b), std::nullopt, false, true,
                                                        std::nullopt));
  const int64_t b = xz.size(0), l = xz.size(2);
  // conv_out is channel-contiguous: its (b l, d) transpose is a row-major view.
  const Tensor x_dbl = gemm(conv_out.transpose(1, 2).reshape({b * l, d}), x_proj_w.t())
                           .view({b, l, R + 2 * N});
  const Tensor delta = gemm(x_dbl.view({b * l, R + 2 * N}).narrow(1, 0, R), dt_proj_w.t())
                           .view({b, l, d}).transpose(1, 2);  // (b, d, l) view
  const Tensor Bk = x_dbl.narrow(-1, R, N).unsqueeze(1), Ck = x_dbl.narrow(-1, R + N, N).unsqueeze(1);
  auto r = scan_fwd_impl(name, conv_out, delta, A.contiguous(), Bk, Ck, f32c(D), opt(z),
                         f32c(delta_bias), softplus, true);
  const Tensor& y = std::get<0>(r);
  const Tensor out = has(out_proj_b)
      ? at::linear(y.transpose(1, 2), out_proj_w, f32c(out_proj_b))
      : gemm(y.transpose(1, 2).reshape({b * l, d}), out_proj_w.t()).view({b, l, out_proj_w.size(0)});
  return {out, conv_out, x_dbl, delta, std::get<2>(r), std::get<3>(r), y};
}

// Gradients (dxz, dconv_w, dconv_b, dx_proj_w, ddt_proj_w, dout_proj_w,
// dout_proj_b, dA, dD, ddelta_bias); those of absent optional inputs are
// empty tensors.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor>
mamba_inner_bwd(const Tensor& dout, const Tensor& xz, const Tensor& conv_w, const optional<Tensor>& conv_b,
                const Tensor& x_proj_w, const Tensor& dt_proj_w, const Tensor& out_proj_w,
                bool has_out_b, const Tensor& A, const optional<Tensor>& D,
                const optional<Tensor>& delta_bias, bool softplus, const Tensor& conv_out,
                const Tensor& x_dbl, const Tensor& delta, const Tensor& ckpt, const Tensor& ysave,
                const Tensor& y) {
  const char* name = "mamba_cpu::mamba_inner_bwd";
  check_inner(name, xz, conv_w, x_proj_w, dt_proj_w, out_proj_w, A);
  c10::DeviceGuard guard(xz.device());
  const int64_t b = xz.size(0), d2 = xz.size(1), l = xz.size(2), d = d2 / 2;
  const int64_t R = dt_proj_w.size(1), N = A.size(1);
  const Tensor x = xz.narrow(1, 0, d), z = xz.narrow(1, d, d);
  const Tensor w2 = conv_w.reshape({d, -1}).contiguous();
  const Tensor g = dout.contiguous();
  const Tensor g2 = g.reshape({-1, g.size(-1)});
  // out_proj
  const Tensor y2 = y.transpose(1, 2).reshape({-1, d});
  const Tensor d_out_proj_w = gemm(g2.t(), y2);
  const Tensor d_out_proj_b = has_out_b ? g2.sum(0) : at::empty({0}, g.options());
  const Tensor dy = gemm(g2, out_proj_w).view({b, l, d}).transpose(1, 2);  // (b, d, l), channel-contiguous
  // scan; dz goes straight into its half of the (b, l, 2d) input gradient
  Tensor dxz = at::empty({b, l, d2}, xz.options());
  const Tensor dz_view = dxz.narrow(2, d, d).transpose(1, 2);
  const Tensor Bk = x_dbl.narrow(-1, R, N).unsqueeze(1), Ck = x_dbl.narrow(-1, R + N, N).unsqueeze(1);
  Grads8 gs = scan_bwd_impl(name, conv_out, delta, A.contiguous(), Bk, Ck, f32c(D), opt(z),
                            f32c(delta_bias), softplus, dy, std::nullopt, ckpt, ysave, &dz_view);
  const Tensor& du = std::get<0>(gs);
  const Tensor ddelta_bl = std::get<1>(gs).transpose(1, 2);  // (b, l, d)
  // dt_proj: delta = dt_in @ dt_proj_w^T
  const Tensor ddelta2 = ddelta_bl.reshape({-1, d});
  const Tensor dt_in2 = x_dbl.view({b * l, R + 2 * N}).narrow(1, 0, R);
  const Tensor d_dt_proj_w = gemm(ddelta2.t(), dt_in2);
  // x_proj output gradient (b * l, R + 2N): d_dt_in, dB, dC side by side
  Tensor dx_dbl = at::empty({b * l, R + 2 * N}, xz.options());
  gemm_into(ddelta2, dt_proj_w, dx_dbl.narrow(1, 0, R), 0.f);
  dx_dbl.narrow(1, R, N).copy_(std::get<3>(gs).select(1, 0).reshape({-1, N}));
  dx_dbl.narrow(1, R + N, N).copy_(std::get<4>(gs).select(1, 0).reshape({-1, N}));
  const Tensor conv2 = conv_out.transpose(1, 2).reshape({-1, d});
  const Tensor d_x_proj_w = gemm(dx_dbl.t(), conv2);
  // dconv = du + dx_dbl @ x_proj_w, accumulated into du's own (b l, d) rows
  const Tensor du2 = du.transpose(1, 2).reshape({-1, d});
  TORCH_CHECK(du2.is_contiguous(), name, ": unexpected du layout");
  gemm_into(dx_dbl, x_proj_w, du2, 1.f);
  const Tensor dconv = du2.view({b, l, d});
  // conv; dx goes straight into its half of the input gradient
  const Tensor dx_view = dxz.narrow(2, 0, d).transpose(1, 2);
  auto cg = conv_bwd_impl(x, w2, f32c(conv_b), std::nullopt, dconv.transpose(1, 2), std::nullopt, true,
                          std::nullopt, &dx_view);
  return {dxz.transpose(1, 2), std::get<1>(cg).view(conv_w.sizes()), std::get<2>(cg), d_x_proj_w,
          d_dt_proj_w, d_out_proj_w, d_out_proj_b, std::get<2>(gs), std::get<5>(gs), std::get<7>(gs)};
}

// ---- selective state update ---------------------------------------------------------

// One decode step in either layout of the reference
// (ops/selective_state_update.py:5-57): Mamba-1 state (b, dim, n), x/dt/z
// (b, dim), A (dim, n), B/C (b, n), D/dt_bias (dim); or Mamba-2 state
// (b, h, p, n), x/dt/z (b, h, p), A (h, p, n), B/C (b, g, n), D/dt_bias (h, p).
// The Mamba-1 layout is the head layout with one head, passed through strides
// without any reshaping op.
Tensor selective_state_update(Tensor& state, const Tensor& x, const Tensor& dt, const Tensor& A_in,
                              const Tensor& B_in, const Tensor& C_in, const optional<Tensor>& D_in,
                              const optional<Tensor>& z, const optional<Tensor>& dt_bias_in,
                              bool dt_softplus, const optional<Tensor>& state_batch_indices) {
  const char* name = "mamba_cpu::selective_state_update";
  check_index(name, "state_batch_indices", state_batch_indices, x.size(0));
  for (const optional<Tensor>& t : {opt(state), opt(x), opt(dt), opt(A_in), opt(B_in), opt(C_in), D_in,
                                    z, dt_bias_in})
    check_gpu(name, t);
  TORCH_CHECK_VALUE(x_dtype(x.scalar_type()) && dt.scalar_type() == x.scalar_type() &&
                        (!has(z) || z->scalar_type() == x.scalar_type()),
                    name, " expects x, dt and z of one dtype among float32, bfloat16, float16");
  TORCH_CHECK_VALUE(x_dtype(state.scalar_type()), name,
                    " expects a float32, bfloat16 or float16 state");
  const bool heads = state.dim() == 4;
  TORCH_CHECK_VALUE((heads && x.dim() == 3) || (state.dim() == 3 && x.dim() == 2), name,
                    " expects state (b, dim, n) with x (b, dim), or state (b, h, p, n) with x (b, h, p)");
  TORCH_CHECK_VALUE(has(state_batch_indices) || state.size(0) == x.size(0), name,
                    " expects state and x of one batch, or state_batch_indices");
  const int64_t b = x.size(0), h = heads ? state.size(1) : 1, p = heads ? state.size(2) : state.size(1);
  const int64_t n = state.size(-1);
  TORCH_CHECK_VALUE(state.stride(-1) == 1 || n == 1, name, " expects unit stride along dstate");
  const bool x_ok = heads ? (x.size(1) == h && x.size(2) == p) : x.size(1) == p;
  TORCH_CHECK_VALUE(x_ok && dt.sizes() == x.sizes() && (!has(z) || z->sizes() == x.sizes()), name,
                    " expects x, dt and z shaped like the state without dstate");
  auto unit_last = [](const Tensor& t) {
    const Tensor f = t.to(at::kFloat);
    return (f.stride(-1) == 1 || f.size(-1) == 1) ? f : f.contiguous();
  };
  // float32 parameters are read through their own strides (the Mamba-2 step
  // passes A, D and dt_bias expanded from per-head values); others are cast.
  auto f32 = [](const Tensor& t) { return t.scalar_type() == at::kFloat ? t : t.to(at::kFloat); };
  auto f32o = [&](const optional<Tensor>& t) { return has(t) ? optional<Tensor>(f32(*t)) : optional<Tensor>(); };
  const Tensor A = f32(A_in), B = unit_last(B_in), C = unit_last(C_in);
  const optional<Tensor> D = f32o(D_in), dt_bias = f32o(dt_bias_in);
  TORCH_CHECK_VALUE(heads ? (A.dim() == 3 && A.size(0) == h && A.size(1) == p && A.size(2) == n)
                          : (A.dim() == 2 && A.size(0) == p && A.size(1) == n),
                    name, " expects A of shape (dim, dstate) or (nheads, headdim, dstate)");
  const int64_t g = heads ? B.size(1) : 1;
  for (const Tensor* X : {&B, &C}) {
    const bool ok = heads ? (X->dim() == 3 && X->size(0) == b && X->size(1) == g && X->size(2) == n)
                          : (X->dim() == 2 && X->size(0) == b && X->size(1) == n);
    TORCH_CHECK_VALUE(ok && (X->stride(-1) == 1 || n == 1), name,
                      " expects B and C of shape (batch, [ngroups,] dstate), unit dstate stride");
  }
  for (const optional<Tensor>& t : {D, dt_bias})
    TORCH_CHECK_VALUE(!has(t) || (heads ? (t->dim() == 2 && t->size(0) == h && t->size(1) == p)
                                        : (t->dim() == 1 && t->size(0) == p)),
                      name, " expects D and dt_bias of shape (dim,) or (nheads, headdim)");
  c10::DeviceGuard guard(x.device());
  Tensor out = at::empty(x.sizes(), x.options());
  mcpu_state_update_args a;
  std::memset(&a, 0, sizeof(a));
  a.state = state.data_ptr();
  a.x = x.data_ptr();
  a.dt = dt.data_ptr();
  a.A = static_cast<const float*>(A.data_ptr());
  a.B = static_cast<const float*>(B.data_ptr());
  a.C = static_cast<const float*>(C.data_ptr());
  a.D = fptr(D);
  a.z = ptr(z);
  a.dt_bias = fptr(dt_bias);
  a.out = out.data_ptr();
  a.batch = b;
  a.nheads = h;
  a.headdim = p;
  a.dstate = n;
  a.ngroups = g;
  a.dt_softplus = dt_softplus ? 1 : 0;
  a.dtype = dtype_tag(x.scalar_type());
  a.state_dtype = dtype_tag(state.scalar_type());
  // Strides over (batch, head, headdim); the Mamba-1 layout has one head.
  auto s3 = [&](int64_t (&d)[3], const Tensor& t) {
    d[0] = t.stride(0);
    d[1] = heads ? t.stride(1) : 0;
    d[2] = t.stride(heads ? 2 : 1);
  };
  s3(a.state_stride, state);
  s3(a.x_stride, x);
  s3(a.dt_stride, dt);
  if (has(z)) s3(a.z_stride, *z);
  a.B_stride[0] = B.stride(0);
  a.B_stride[1] = heads ? B.stride(1) : 0;
  a.C_stride[0] = C.stride(0);
  a.C_stride[1] = heads ? C.stride(1) : 0;
  a.state_batch_indices =
      has(state_batch_indices) ? static_cast<const int32_t*>(state_batch_indices->data_ptr()) : nullptr;
  a.state_batch = state.size(0);
  a.param_strides = 1;
  a.A_stride[0] = heads ? A.stride(0) : 0;
  a.A_stride[1] = A.stride(heads ? 1 : 0);
  a.A_stride[2] = A.stride(heads ? 2 : 1);
  auto s2 = [&](int64_t (&d)[2], const optional<Tensor>& t) {
    if (!has(t)) return;
    d[0] = heads ? t->stride(0) : 0;
    d[1] = t->stride(heads ? 1 : 0);
  };
  s2(a.D_stride, D);
  s2(a.dt_bias_stride, dt_bias);
  check_rc(mcpu_selective_state_update(&a, stream_of(x)), name);
  return out;
}

// The two in-place ops record their mutation for autograd's version counters
// (what torch.library does for a Python custom op with mutates_args).
Tensor causal_conv1d_update_inplace(const Tensor& x, Tensor& conv_state, const Tensor& weight,
                                    const optional<Tensor>& bias, bool silu,
                                    const optional<Tensor>& cache_seqlens,
                                    const optional<Tensor>& conv_state_indices) {
  Tensor out;
  {
    at::AutoDispatchBelowADInplaceOrView below;
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("mamba_cpu::causal_conv1d_update", "")
                         .typed<decltype(causal_conv1d_update)>();
    out = op.call(x, conv_state, weight, bias, silu, cache_seqlens, conv_state_indices);
  }
  conv_state.unsafeGetTensorImpl()->bump_version();
  return out;
}

Tensor selective_state_update_inplace(Tensor& state, const Tensor& x, const Tensor& dt,
                                      const Tensor& A, const Tensor& B, const Tensor& C,
                                      const optional<Tensor>& D, const optional<Tensor>& z,
                                      const optional<Tensor>& dt_bias, bool dt_softplus,
                                      const optional<Tensor>& state_batch_indices) {
  Tensor out;
  {
    at::AutoDispatchBelowADInplaceOrView below;
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("mamba_cpu::selective_state_update", "")
                         .typed<decltype(selective_state_update)>();
    out = op.call(state, x, dt, A, B, C, D, z, dt_bias, dt_softplus, state_batch_indices);
  }
  state.unsafeGetTensorImpl()->bump_version();
  return out;
}

// ---- Mamba-2 SSD scan ------------------------------------------------------------
//
// mamba_chunk_scan_combined's forward and backward over mcpu_ssd_fwd / _bwd.
// Layouts as the C ABI takes them (all contiguous): x, z (batch, seqlen,
// nheads, headdim) in one storage type; dt (batch, seqlen, nheads) float32;
// A, dt_bias (nheads) float32; B, C (batch, seqlen, ngroups, dstate) in x's
// type; D (nheads, headdim) float32; initial_states (batch, nheads, headdim,
// dstate) float32; seq_idx (batch, seqlen) int32 packed-sequence ids, not
// decreasing along the sequence. The Python wrapper
// (mamba_cpu/ops/ssd_combined.py) brings its arguments to these.

mcpu_ssd_args ssd_args(const char* name, const Tensor& x, const Tensor& dt, const Tensor& A,
                       const Tensor& B, const Tensor& C, const optional<Tensor>& D,
                       const optional<Tensor>& z, const optional<Tensor>& dt_bias,
                       const optional<Tensor>& init, bool softplus, double lo, double hi,
                       int64_t head_block, int64_t chunk_pass, const optional<Tensor>& seq_idx) {
  for (const optional<Tensor>& t : {opt(x), opt(dt), opt(A), opt(B), opt(C), D, z, dt_bias, init, seq_idx})
    check_gpu(name, t);
  TORCH_CHECK_VALUE(x.dim() == 4 && x_dtype(x.scalar_type()) && x.is_contiguous(), name,
                    " expects a contiguous x (batch, seqlen, nheads, headdim) in float32, bfloat16 or float16");
  const int64_t b = x.size(0), l = x.size(1), h = x.size(2), p = x.size(3);
  TORCH_CHECK_VALUE(dt.scalar_type() == at::kFloat && dt.is_contiguous() && dt.dim() == 3 &&
                        dt.size(0) == b && dt.size(1) == l && dt.size(2) == h,
                    name, " expects a contiguous float32 dt (batch, seqlen, nheads)");
  TORCH_CHECK_VALUE(A.scalar_type() == at::kFloat && A.dim() == 1 && A.size(0) == h && A.is_contiguous(), name,
                    " expects a float32 A of shape (nheads,)");
  for (const Tensor* X : {&B, &C})
    TORCH_CHECK_VALUE(X->dim() == 4 && X->size(0) == b && X->size(1) == l && X->scalar_type() == x.scalar_type() &&
                          X->is_contiguous(),
                      name, " expects contiguous B and C (batch, seqlen, ngroups, dstate) in x's dtype");
  TORCH_CHECK_VALUE(B.sizes() == C.sizes(), name, " expects B and C of one shape");
  TORCH_CHECK_VALUE(!has(D) || (D->scalar_type() == at::kFloat && D->dim() == 2 && D->size(0) == h &&
                                D->size(1) == p && D->is_contiguous()),
                    name, " expects a float32 D of shape (nheads, headdim)");
  TORCH_CHECK_VALUE(!has(z) || (z->sizes() == x.sizes() && z->scalar_type() == x.scalar_type() && z->is_contiguous()),
                    name, " expects a contiguous z like x");
  TORCH_CHECK_VALUE(!has(dt_bias) || (dt_bias->scalar_type() == at::kFloat && dt_bias->dim() == 1 &&
                                      dt_bias->size(0) == h && dt_bias->is_contiguous()),
                    name, " expects a float32 dt_bias of shape (nheads,)");
  TORCH_CHECK_VALUE(!has(init) || (init->scalar_type() == at::kFloat && init->dim() == 4 && init->size(0) == b &&
                                   init->size(1) == h && init->size(2) == p && init->size(3) == B.size(3) &&
                                   init->is_contiguous()),
                    name, " expects float32 initial_states (batch, nheads, headdim, dstate)");
  TORCH_CHECK_VALUE(!has(seq_idx) || (seq_idx->scalar_type() == at::kInt && seq_idx->dim() == 2 &&
                                      seq_idx->size(0) == b && seq_idx->size(1) == l && seq_idx->is_contiguous()),
                    name, " expects a contiguous int32 seq_idx (batch, seqlen)");
  mcpu_ssd_args a;
  std::memset(&a, 0, sizeof(a));
  a.x = x.data_ptr();
  a.dt = static_cast<const float*>(dt.data_ptr());
  a.A = static_cast<const float*>(A.data_ptr());
  a.B = B.data_ptr();
  a.C = C.data_ptr();
  a.D = fptr(D);
  a.z = ptr(z);
  a.dt_bias = fptr(dt_bias);
  a.initial_states = fptr(init);
  a.batch = b;
  a.seqlen = l;
  a.nheads = h;
  a.headdim = p;
  a.ngroups = B.size(2);
  a.dstate = B.size(3);
  a.dtype = dtype_tag(x.scalar_type());
  a.dt_softplus = softplus ? 1 : 0;
  a.dt_limit_lo = static_cast<float>(lo);
  a.dt_limit_hi = static_cast<float>(hi);
  a.head_block = static_cast<int32_t>(head_block);
  a.chunk_pass = static_cast<int32_t>(chunk_pass);
  a.seq_idx = has(seq_idx) ? static_cast<const int32_t*>(seq_idx->data_ptr()) : nullptr;
  return a;
}

std::tuple<Tensor, Tensor, Tensor, Tensor> ssd_fwd(const Tensor& x, const Tensor& dt, const Tensor& A,
                                                   const Tensor& B, const Tensor& C, const optional<Tensor>& D,
                                                   const optional<Tensor>& z, const optional<Tensor>& dt_bias,
                                                   const optional<Tensor>& init, bool softplus, double lo,
                                                   double hi, bool save_for_backward, int64_t head_block,
                                                   int64_t chunk_pass, const optional<Tensor>& seq_idx) {
  const char* name = "mamba_cpu::ssd_fwd";
  mcpu_ssd_args a =
      ssd_args(name, x, dt, A, B, C, D, z, dt_bias, init, softplus, lo, hi, head_block, chunk_pass, seq_idx);
  c10::DeviceGuard guard(x.device());
  Tensor out = at::empty(x.sizes(), x.options());
  Tensor fin = at::empty({a.batch, a.nheads, a.headdim, a.dstate}, x.options().dtype(at::kFloat));
  Tensor ysave = (save_for_backward && has(z)) ? at::empty(x.sizes(), x.options()) : x.new_empty({0});
  // 0 for an empty sequence; for arguments the library rejects, the
  // forward call below reports why.
  const size_t nsaved = mcpu_ssd_saved_size(&a);
  Tensor saved = at::empty({static_cast<int64_t>(nsaved)}, x.options().dtype(at::kByte));
  a.out = out.data_ptr();
  a.final_states = static_cast<float*>(fin.data_ptr());
  a.ysave = ysave.numel() ? ysave.data_ptr() : nullptr;
  check_rc(mcpu_ssd_fwd(&a, saved.data_ptr(), nsaved, stream_of(x)), name);
  return {out, fin, saved, ysave};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> ssd_bwd(
    const Tensor& dout, const optional<Tensor>& dfinal, const Tensor& x, const Tensor& dt, const Tensor& A,
    const Tensor& B, const Tensor& C, const optional<Tensor>& D, const optional<Tensor>& z,
    const optional<Tensor>& dt_bias, const optional<Tensor>& init, bool softplus, double lo, double hi,
    const Tensor& saved, const Tensor& ysave, int64_t head_block, int64_t chunk_pass,
    const optional<Tensor>& seq_idx) {
  const char* name = "mamba_cpu::ssd_bwd";
  mcpu_ssd_args a =
      ssd_args(name, x, dt, A, B, C, D, z, dt_bias, init, softplus, lo, hi, head_block, chunk_pass, seq_idx);
  check_gpu(name, opt(dout));
  check_gpu(name, dfinal);
  TORCH_CHECK_VALUE(dout.sizes() == x.sizes() && dout.scalar_type() == x.scalar_type() && dout.is_contiguous(),
                    name, " expects a contiguous dout like x");
  TORCH_CHECK_VALUE(!has(dfinal) || (dfinal->scalar_type() == at::kFloat && dfinal->is_contiguous() &&
                                     dfinal->dim() == 4 && dfinal->size(0) == a.batch &&
                                     dfinal->size(1) == a.nheads && dfinal->size(2) == a.headdim &&
                                     dfinal->size(3) == a.dstate),
                    name, " expects a float32 dfinal_states (batch, nheads, headdim, dstate)");
  const size_t nsaved = mcpu_ssd_saved_size(&a);
  TORCH_CHECK_VALUE(saved.scalar_type() == at::kByte && static_cast<size_t>(saved.numel()) >= nsaved && saved.is_cuda(),
                    name, " expects the forward's saved buffer");
  TORCH_CHECK_VALUE(!has(z) || (ysave.sizes() == x.sizes() && ysave.scalar_type() == x.scalar_type()), name,
                    " expects the forward's ysave when z is given");
  c10::DeviceGuard guard(x.device());
  const auto f32 = x.options().dtype(at::kFloat);
  Tensor dx = at::empty(x.sizes(), x.options());
  Tensor ddt = at::empty(dt.sizes(), f32);
  Tensor dA = at::empty({a.nheads}, f32);
  Tensor dB = at::empty(B.sizes(), f32);
  Tensor dC = at::empty(C.sizes(), f32);
  Tensor dD = has(D) ? at::empty(D->sizes(), f32) : A.new_empty({0});
  Tensor dz = has(z) ? at::empty(x.sizes(), x.options()) : x.new_empty({0});
  Tensor dbias = has(dt_bias) ? at::empty({a.nheads}, f32) : A.new_empty({0});
  Tensor dinit = has(init) ? at::empty(init->sizes(), f32) : A.new_empty({0});
  a.ysave = has(z) ? ysave.data_ptr() : nullptr;
  a.dout = dout.data_ptr();
  a.dfinal_states = fptr(dfinal);
  a.dx = dx.data_ptr();
  a.ddt = static_cast<float*>(ddt.data_ptr());
  a.dA = static_cast<float*>(dA.data_ptr());
  a.dB = static_cast<float*>(dB.data_ptr());
  a.dC = static_cast<float*>(dC.data_ptr());
  a.dD = has(D) ? static_cast<float*>(dD.data_ptr()) : nullptr;
  a.dz = has(z) ? dz.data_ptr() : nullptr;
  a.ddt_bias = has(dt_bias) ? static_cast<float*>(dbias.data_ptr()) : nullptr;
  a.dinitial_states = has(init) ? static_cast<float*>(dinit.data_ptr()) : nullptr;
  const size_t nws = mcpu_ssd_bwd_workspace_size(&a);
  Tensor ws = at::empty({static_cast<int64_t>(nws)}, x.options().dtype(at::kByte));
  check_rc(mcpu_ssd_bwd(&a, saved.data_ptr(), saved.numel(), ws.data_ptr(), nws, stream_of(x)), name);
  return {dx, ddt, dA, dB, dC, dD, dz, dbias, dinit};
}

// Per-sequence final states (nseqs, nheads, headdim, dstate) float32 of the
// packed sequences of batch row 0, from the forward's saved buffer;
// cu_seqlens (nseqs + 1) int32 offsets.
Tensor ssd_varlen_states(const Tensor& x, const Tensor& dt, const Tensor& A, const Tensor& B, const Tensor& C,
                         const optional<Tensor>& D, const optional<Tensor>& z, const optional<Tensor>& dt_bias,
                         const optional<Tensor>& init, bool softplus, double lo, double hi, const Tensor& saved,
                         const Tensor& cu_seqlens, int64_t head_block, int64_t chunk_pass,
                         const optional<Tensor>& seq_idx) {
  const char* name = "mamba_cpu::ssd_varlen_states";
  mcpu_ssd_args a =
      ssd_args(name, x, dt, A, B, C, D, z, dt_bias, init, softplus, lo, hi, head_block, chunk_pass, seq_idx);
  check_gpu(name, opt(cu_seqlens));
  TORCH_CHECK_VALUE(cu_seqlens.scalar_type() == at::kInt && cu_seqlens.dim() == 1 && cu_seqlens.numel() >= 1 &&
                        cu_seqlens.is_contiguous(),
                    name, " expects contiguous int32 cu_seqlens (nseqs + 1)");
  TORCH_CHECK_VALUE(saved.scalar_type() == at::kByte && saved.is_cuda(), name, " expects the forward's saved buffer");
  c10::DeviceGuard guard(x.device());
  const int64_t nseqs = cu_seqlens.numel() - 1;
  Tensor out = at::empty({nseqs, a.nheads, a.headdim, a.dstate}, x.options().dtype(at::kFloat));
  check_rc(mcpu_ssd_varlen_states(&a, saved.data_ptr(), saved.numel(),
                                  static_cast<const int32_t*>(cu_seqlens.data_ptr()), nseqs,
                                  static_cast<float*>(out.data_ptr()), stream_of(x)),
           name);
  return out;
}

// ---- fused single-token block step ----------------------------------------------

// One decode step of a Mamba-1 block (mcpu_mixer_step): hidden (batch,
// d_model) -> out (batch, d_model), conv_state (batch, d_inner, state_len) and
// ssm_state (batch, d_inner, dstate) updated in place. Weights as nn.Linear /
// nn.Conv1d hold them (conv weight (d_inner, width)); dt_bias, A (= -exp(A_log))
// and D float32. out is float32 when the residual is (add_residual with a
// float32 residual), else the weights' dtype.
Tensor mixer_step(const Tensor& hidden, const optional<Tensor>& norm_weight, double eps, bool add_residual,
                  bool residual_in_fp32, const Tensor& in_w, const optional<Tensor>& in_b, const Tensor& conv_w,
                  const optional<Tensor>& conv_b, Tensor& conv_state, const Tensor& x_w, const Tensor& dt_w,
                  const optional<Tensor>& dt_b, const Tensor& A, const optional<Tensor>& D, Tensor& ssm_state,
                  const Tensor& out_w, const optional<Tensor>& out_b) {
  const char* name = "mamba_cpu::mixer_step";
  for (const optional<Tensor>& t : {opt(hidden), norm_weight, opt(in_w), in_b, opt(conv_w), conv_b,
                                    opt(conv_state), opt(x_w), opt(dt_w), dt_b, opt(A), D, opt(ssm_state),
                                    opt(out_w), out_b})
    check_gpu(name, t);
  const auto T = in_w.scalar_type();
  TORCH_CHECK_VALUE(x_dtype(T), name, " expects float32, bfloat16 or float16 weights");
  for (const optional<Tensor>& t : {norm_weight, in_b, opt(conv_w), conv_b, opt(conv_state), opt(x_w),
                                    opt(dt_w), opt(out_w), out_b})
    TORCH_CHECK_VALUE(!has(t) || (t->scalar_type() == T && t->is_contiguous()), name,
                      " expects contiguous weights, biases and conv state of one dtype");
  for (const optional<Tensor>& t : {dt_b, opt(A), D})
    TORCH_CHECK_VALUE(!has(t) || (t->scalar_type() == at::kFloat && t->is_contiguous()), name,
                      " expects contiguous float32 dt_bias, A and D");
  TORCH_CHECK_VALUE(hidden.dim() == 2 && hidden.is_contiguous() &&
                        (hidden.scalar_type() == T || hidden.scalar_type() == at::kFloat),
                    name, " expects a contiguous hidden (batch, d_model) in the weights' dtype or float32");
  const int64_t b = hidden.size(0), dm = hidden.size(1);
  TORCH_CHECK_VALUE(in_w.dim() == 2 && in_w.size(1) == dm && in_w.size(0) % 2 == 0, name,
                    " expects in_proj weight (2 d_inner, d_model)");
  const int64_t di = in_w.size(0) / 2;
  TORCH_CHECK_VALUE(conv_w.dim() == 2 && conv_w.size(0) == di, name, " expects conv weight (d_inner, width)");
  TORCH_CHECK_VALUE(conv_state.dim() == 3 && conv_state.size(0) == b && conv_state.size(1) == di, name,
                    " expects conv_state (batch, d_inner, state_len)");
  TORCH_CHECK_VALUE(A.dim() == 2 && A.size(0) == di, name, " expects A (d_inner, dstate)");
  const int64_t N = A.size(1);
  TORCH_CHECK_VALUE(dt_w.dim() == 2 && dt_w.size(0) == di, name, " expects dt_proj weight (d_inner, dt_rank)");
  const int64_t R = dt_w.size(1);
  TORCH_CHECK_VALUE(x_w.dim() == 2 && x_w.size(0) == R + 2 * N && x_w.size(1) == di, name,
                    " expects x_proj weight (dt_rank + 2 dstate, d_inner)");
  TORCH_CHECK_VALUE(out_w.dim() == 2 && out_w.size(0) == dm && out_w.size(1) == di, name,
                    " expects out_proj weight (d_model, d_inner)");
  TORCH_CHECK_VALUE(ssm_state.dim() == 3 && ssm_state.size(0) == b && ssm_state.size(1) == di &&
                        ssm_state.size(2) == N && ssm_state.is_contiguous() && x_dtype(ssm_state.scalar_type()),
                    name, " expects a contiguous ssm_state (batch, d_inner, dstate)");
  TORCH_CHECK_VALUE((!has(norm_weight) || norm_weight->numel() == dm) && (!has(in_b) || in_b->numel() == 2 * di) &&
                        (!has(conv_b) || conv_b->numel() == di) && (!has(dt_b) || dt_b->numel() == di) &&
                        (!has(D) || D->numel() == di) && (!has(out_b) || out_b->numel() == dm),
                    name, " expects bias and norm vectors of their layer's width");
  const bool res32 = add_residual && (residual_in_fp32 || hidden.scalar_type() == at::kFloat);
  c10::DeviceGuard guard(hidden.device());
  Tensor out = at::empty({b, dm}, hidden.options().dtype(res32 ? at::kFloat : T));
  mcpu_mixer_step_args a;
  std::memset(&a, 0, sizeof(a));
  a.hidden = hidden.data_ptr();
  a.norm_weight = ptr(norm_weight);
  a.in_w = in_w.data_ptr();
  a.in_b = ptr(in_b);
  a.conv_w = conv_w.data_ptr();
  a.conv_b = ptr(conv_b);
  a.conv_state = conv_state.data_ptr();
  a.x_w = x_w.data_ptr();
  a.dt_w = dt_w.data_ptr();
  a.dt_b = fptr(dt_b);
  a.A = static_cast<const float*>(A.data_ptr());
  a.D = fptr(D);
  a.ssm_state = ssm_state.data_ptr();
  a.out_w = out_w.data_ptr();
  a.out_b = ptr(out_b);
  a.out = out.data_ptr();
  a.batch = b;
  a.d_model = dm;
  a.d_inner = di;
  a.dt_rank = R;
  a.dstate = N;
  a.width = conv_w.size(1);
  a.state_len = conv_state.size(2);
  a.norm_eps = static_cast<float>(eps);
  a.add_residual = add_residual ? 1 : 0;
  a.residual_in_fp32 = residual_in_fp32 ? 1 : 0;
  a.dtype = dtype_tag(T);
  a.hidden_dtype = dtype_tag(hidden.scalar_type());
  a.state_dtype = dtype_tag(ssm_state.scalar_type());
  a.out_dtype = dtype_tag(out.scalar_type());
  const size_t nws = mcpu_mixer_step_workspace_size(&a);
  Tensor ws = at::empty({static_cast<int64_t>(nws)}, hidden.options().dtype(at::kByte));
  check_rc(mcpu_mixer_step(&a, ws.data_ptr(), nws, stream_of(hidden)), name);
  return out;
}

// Final norm and output head of a decode step (mcpu_norm_linear): hidden
// (batch, d_in) in the weights' dtype or float32 -> Linear(RMSNorm(hidden))
// (batch, d_out), float32 when out_float32, else the weights' dtype.
Tensor norm_linear(const Tensor& hidden, const optional<Tensor>& norm_weight, double eps, const Tensor& weight,
                   const optional<Tensor>& bias, bool out_float32) {
  const char* name = "mamba_cpu::norm_linear";
  for (const optional<Tensor>& t : {opt(hidden), norm_weight, opt(weight), bias}) check_gpu(name, t);
  const auto T = weight.scalar_type();
  TORCH_CHECK_VALUE(x_dtype(T), name, " expects float32, bfloat16 or float16 weights");
  for (const optional<Tensor>& t : {norm_weight, opt(weight), bias})
    TORCH_CHECK_VALUE(!has(t) || (t->scalar_type() == T && t->is_contiguous()), name,
                      " expects contiguous weight, bias and norm weight of one dtype");
  TORCH_CHECK_VALUE(hidden.dim() == 2 && hidden.is_contiguous() &&
                        (hidden.scalar_type() == T || hidden.scalar_type() == at::kFloat),
                    name, " expects a contiguous hidden (batch, d_in) in the weights' dtype or float32");
  const int64_t b = hidden.size(0), din = hidden.size(1);
  TORCH_CHECK_VALUE(weight.dim() == 2 && weight.size(1) == din, name, " expects weight (d_out, d_in)");
  const int64_t dout = weight.size(0);
  TORCH_CHECK_VALUE((!has(norm_weight) || norm_weight->numel() == din) && (!has(bias) || bias->numel() == dout),
                    name, " expects norm weight (d_in) and bias (d_out)");
  c10::DeviceGuard guard(hidden.device());
  Tensor out = at::empty({b, dout}, hidden.options().dtype(out_float32 ? at::kFloat : T));
  if (b == 0 || dout == 0) return out;
  mcpu_norm_linear_args a;
  std::memset(&a, 0, sizeof(a));
  a.hidden = hidden.data_ptr();
  a.norm_weight = ptr(norm_weight);
  a.weight = weight.data_ptr();
  a.bias = ptr(bias);
  a.out = out.data_ptr();
  a.batch = b;
  a.d_in = din;
  a.d_out = dout;
  a.norm_eps = static_cast<float>(eps);
  a.dtype = dtype_tag(T);
  a.hidden_dtype = dtype_tag(hidden.scalar_type());
  a.out_dtype = dtype_tag(out.scalar_type());
  check_rc(mcpu_norm_linear(&a, stream_of(hidden)), name);
  return out;
}

// One decode step of a Mamba-2 block (mcpu_mamba2_step): hidden (batch,
// d_model) -> out (batch, d_model), conv_state (batch, conv_dim, state_len)
// and ssm_state (batch, nheads, headdim, dstate) updated in place. Sizes come
// from the tensors: d_inner from the gated norm's weight, nheads from A,
// headdim and dstate from ssm_state, ngroups from the conv's width
// conv_dim = d_inner + 2 ngroups dstate. dt_bias, A (= -exp(A_log)) and D
// float32 per head.
Tensor mamba2_step(const Tensor& hidden, const optional<Tensor>& norm_weight, double eps, bool add_residual,
                   bool residual_in_fp32, const Tensor& in_w, const optional<Tensor>& in_b, const Tensor& conv_w,
                   const optional<Tensor>& conv_b, Tensor& conv_state, const optional<Tensor>& dt_bias,
                   const Tensor& A, const optional<Tensor>& D, Tensor& ssm_state, const Tensor& gate_norm_w,
                   double gate_eps, const Tensor& out_w, const optional<Tensor>& out_b) {
  const char* name = "mamba_cpu::mamba2_step";
  for (const optional<Tensor>& t : {opt(hidden), norm_weight, opt(in_w), in_b, opt(conv_w), conv_b,
                                    opt(conv_state), dt_bias, opt(A), D, opt(ssm_state), opt(gate_norm_w),
                                    opt(out_w), out_b})
    check_gpu(name, t);
  const auto T = in_w.scalar_type();
  TORCH_CHECK_VALUE(x_dtype(T), name, " expects float32, bfloat16 or float16 weights");
  for (const optional<Tensor>& t : {norm_weight, in_b, opt(conv_w), conv_b, opt(conv_state), opt(gate_norm_w),
                                    opt(out_w), out_b})
    TORCH_CHECK_VALUE(!has(t) || (t->scalar_type() == T && t->is_contiguous()), name,
                      " expects contiguous weights, biases and conv state of one dtype");
  for (const optional<Tensor>& t : {dt_bias, opt(A), D})
    TORCH_CHECK_VALUE(!has(t) || (t->scalar_type() == at::kFloat && t->is_contiguous()), name,
                      " expects contiguous float32 dt_bias, A and D");
  TORCH_CHECK_VALUE(hidden.dim() == 2 && hidden.is_contiguous() &&
                        (hidden.scalar_type() == T || hidden.scalar_type() == at::kFloat),
                    name, " expects a contiguous hidden (batch, d_model) in the weights' dtype or float32");
  TORCH_CHECK_VALUE(ssm_state.dim() == 4 && ssm_state.is_contiguous() && x_dtype(ssm_state.scalar_type()), name,
                    " expects a contiguous ssm_state (batch, nheads, headdim, dstate)");
  const int64_t b = hidden.size(0), dm = hidden.size(1), di = gate_norm_w.numel(), nh = A.numel();
  const int64_t hd = ssm_state.size(2), N = ssm_state.size(3);
  TORCH_CHECK_VALUE(conv_w.dim() == 2, name, " expects conv weight (conv_dim, width)");
  const int64_t conv_dim = conv_w.size(0);
  TORCH_CHECK_VALUE(conv_dim > di && (conv_dim - di) % (2 * N) == 0, name,
                    " expects conv_dim = d_inner + 2 ngroups dstate");
  const int64_t ng = (conv_dim - di) / (2 * N);
  TORCH_CHECK_VALUE(ssm_state.size(0) == b && ssm_state.size(1) == nh && nh * hd == di, name,
                    " expects ssm_state (batch, nheads, headdim, dstate) with nheads x headdim = d_inner");
  TORCH_CHECK_VALUE(in_w.dim() == 2 && in_w.size(1) == dm && in_w.size(0) == di + conv_dim + nh, name,
                    " expects in_proj weight (d_inner + conv_dim + nheads, d_model)");
  TORCH_CHECK_VALUE(conv_state.dim() == 3 && conv_state.size(0) == b && conv_state.size(1) == conv_dim, name,
                    " expects conv_state (batch, conv_dim, state_len)");
  TORCH_CHECK_VALUE(out_w.dim() == 2 && out_w.size(0) == dm && out_w.size(1) == di, name,
                    " expects out_proj weight (d_model, d_inner)");
  TORCH_CHECK_VALUE((!has(norm_weight) || norm_weight->numel() == dm) && (!has(in_b) || in_b->numel() == in_w.size(0)) &&
                        (!has(conv_b) || conv_b->numel() == conv_dim) && (!has(dt_bias) || dt_bias->numel() == nh) &&
                        (!has(D) || D->numel() == nh) && (!has(out_b) || out_b->numel() == dm),
                    name, " expects bias and norm vectors of their layer's width");
  const bool res32 = add_residual && (residual_in_fp32 || hidden.scalar_type() == at::kFloat);
  c10::DeviceGuard guard(hidden.device());
  Tensor out = at::empty({b, dm}, hidden.options().dtype(res32 ? at::kFloat : T));
  mcpu_mamba2_step_args a;
  std::memset(&a, 0, sizeof(a));
  a.hidden = hidden.data_ptr();
  a.norm_weight = ptr(norm_weight);
  a.in_w = in_w.data_ptr();
  a.in_b = ptr(in_b);
  a.conv_w = conv_w.data_ptr();
  a.conv_b = ptr(conv_b);
  a.conv_state = conv_state.data_ptr();
  a.dt_bias = fptr(dt_bias);
  a.A = static_cast<const float*>(A.data_ptr());
  a.D = fptr(D);
  a.ssm_state = ssm_state.data_ptr();
  a.gate_norm_weight = gate_norm_w.data_ptr();
  a.out_w = out_w.data_ptr();
  a.out_b = ptr(out_b);
  a.out = out.data_ptr();
  a.batch = b;
  a.d_model = dm;
  a.d_inner = di;
  a.nheads = nh;
  a.headdim = hd;
  a.ngroups = ng;
  a.dstate = N;
  a.width = conv_w.size(1);
  a.state_len = conv_state.size(2);
  a.norm_eps = static_cast<float>(eps);
  a.gate_norm_eps = static_cast<float>(gate_eps);
  a.add_residual = add_residual ? 1 : 0;
  a.residual_in_fp32 = residual_in_fp32 ? 1 : 0;
  a.dtype = dtype_tag(T);
  a.hidden_dtype = dtype_tag(hidden.scalar_type());
  a.state_dtype = dtype_tag(ssm_state.scalar_type());
  a.out_dtype = dtype_tag(out.scalar_type());
  const size_t nws = mcpu_mamba2_step_workspace_size(&a);
  Tensor ws = at::empty({static_cast<int64_t>(nws > 0 ? nws : 1)}, hidden.options().dtype(at::kByte));
  check_rc(mcpu_mamba2_step(&a, ws.data_ptr(), nws, stream_of(hidden)), name);
  return out;
}

Tensor mamba2_step_inplace(const Tensor& hidden, const optional<Tensor>& norm_weight, double eps,
                           bool add_residual, bool residual_in_fp32, const Tensor& in_w,
                           const optional<Tensor>& in_b, const Tensor& conv_w, const optional<Tensor>& conv_b,
                           Tensor& conv_state, const optional<Tensor>& dt_bias, const Tensor& A,
                           const optional<Tensor>& D, Tensor& ssm_state, const Tensor& gate_norm_w,
                           double gate_eps, const Tensor& out_w, const optional<Tensor>& out_b) {
  Tensor out;
  {
    at::AutoDispatchBelowADInplaceOrView below;
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("mamba_cpu::mamba2_step", "")
                         .typed<decltype(mamba2_step)>();
    out = op.call(hidden, norm_weight, eps, add_residual, residual_in_fp32, in_w, in_b, conv_w, conv_b,
                  conv_state, dt_bias, A, D, ssm_state, gate_norm_w, gate_eps, out_w, out_b);
  }
  conv_state.unsafeGetTensorImpl()->bump_version();
  ssm_state.unsafeGetTensorImpl()->bump_version();
  return out;
}

Tensor mixer_step_inplace(const Tensor& hidden, const optional<Tensor>& norm_weight, double eps, bool add_residual,
                          bool residual_in_fp32, const Tensor& in_w, const optional<Tensor>& in_b,
                          const Tensor& conv_w, const optional<Tensor>& conv_b, Tensor& conv_state,
                          const Tensor& x_w, const Tensor& dt_w, const optional<Tensor>& dt_b, const Tensor& A,
                          const optional<Tensor>& D, Tensor& ssm_state, const Tensor& out_w,
                          const optional<Tensor>& out_b) {
  Tensor out;
  {
    at::AutoDispatchBelowADInplaceOrView below;
    static auto op = c10::Dispatcher::singleton()
                         .findSchemaOrThrow("mamba_cpu::mixer_step", "")
                         .typed<decltype(mixer_step)>();
    out = op.call(hidden, norm_weight, eps, add_residual, residual_in_fp32, in_w, in_b, conv_w, conv_b, conv_state,
                  x_w, dt_w, dt_b, A, D, ssm_state, out_w, out_b);
  }
  conv_state.unsafeGetTensorImpl()->bump_version();
  ssm_state.unsafeGetTensorImpl()->bump_version();
  return out;
}

}  // namespace
}  // namespace mcpu_torch

TORCH_LIBRARY(mamba_cpu, m) {
  m.def("ssd_fwd(Tensor x, Tensor dt, Tensor A, Tensor B, Tensor C, Tensor? D, Tensor? z, "
        "Tensor? dt_bias, Tensor? initial_states, bool dt_softplus, float dt_lo, float dt_hi, "
        "bool save_for_backward, int head_block=0, int chunk_pass=0, Tensor? seq_idx=None) -> "
        "(Tensor, Tensor, Tensor, Tensor)");
  m.def("ssd_bwd(Tensor dout, Tensor? dfinal_states, Tensor x, Tensor dt, Tensor A, Tensor B, Tensor C, "
        "Tensor? D, Tensor? z, Tensor? dt_bias, Tensor? initial_states, bool dt_softplus, float dt_lo, "
        "float dt_hi, Tensor saved, Tensor ysave, int head_block=0, int chunk_pass=0, Tensor? seq_idx=None) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("ssd_varlen_states(Tensor x, Tensor dt, Tensor A, Tensor B, Tensor C, Tensor? D, Tensor? z, "
        "Tensor? dt_bias, Tensor? initial_states, bool dt_softplus, float dt_lo, float dt_hi, Tensor saved, "
        "Tensor cu_seqlens, int head_block=0, int chunk_pass=0, Tensor? seq_idx=None) -> Tensor");
  m.def("selective_scan_fwd(Tensor u, Tensor delta, Tensor A, Tensor B, Tensor C, Tensor? D, "
        "Tensor? z, Tensor? delta_bias, bool delta_softplus) -> (Tensor, Tensor)");
  m.def("selective_scan_bwd(Tensor u, Tensor delta, Tensor A, Tensor B, Tensor C, Tensor? D, "
        "Tensor? z, Tensor? delta_bias, bool delta_softplus, Tensor dout, Tensor? dlast_state) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("selective_scan_fwd_ckpt(Tensor u, Tensor delta, Tensor A, Tensor B, Tensor C, Tensor? D, "
        "Tensor? z, Tensor? delta_bias, bool delta_softplus) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("selective_scan_bwd_ckpt(Tensor u, Tensor delta, Tensor A, Tensor B, Tensor C, Tensor? D, "
        "Tensor? z, Tensor? delta_bias, bool delta_softplus, Tensor dout, Tensor? dlast_state, "
        "Tensor ckpt, Tensor ysave) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("selective_scan_cfwd(Tensor u, Tensor delta, Tensor A, Tensor B, Tensor C, Tensor? D, "
        "Tensor? z, Tensor? delta_bias, bool delta_softplus) -> (Tensor, Tensor, Tensor)");
  m.def("selective_scan_cbwd(Tensor u, Tensor delta, Tensor A, Tensor B, Tensor C, Tensor? D, "
        "Tensor? z, Tensor? delta_bias, bool delta_softplus, Tensor dout, Tensor? dlast_state, "
        "Tensor? ckpt) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("mamba_inner_fwd(Tensor xz, Tensor conv1d_weight, Tensor? conv1d_bias, Tensor x_proj_weight, "
        "Tensor delta_proj_weight, Tensor out_proj_weight, Tensor? out_proj_bias, Tensor A, Tensor? D, "
        "Tensor? delta_bias, bool delta_softplus) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("mamba_inner_bwd(Tensor dout, Tensor xz, Tensor conv1d_weight, Tensor? conv1d_bias, "
        "Tensor x_proj_weight, Tensor delta_proj_weight, Tensor out_proj_weight, bool has_out_proj_bias, "
        "Tensor A, Tensor? D, Tensor? delta_bias, bool delta_softplus, Tensor conv_out, Tensor x_dbl, "
        "Tensor delta, Tensor ckpt, Tensor ysave, Tensor y) -> (Tensor, Tensor, Tensor, Tensor, Tensor, "
        "Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("causal_conv1d_fwd(Tensor x, Tensor weight, Tensor? bias, Tensor? initial_states, "
        "bool return_final_states, bool silu, Tensor? seq_idx=None) -> (Tensor, Tensor)");
  m.def("causal_conv1d_bwd(Tensor x, Tensor weight, Tensor? bias, Tensor? initial_states, "
        "Tensor dout, Tensor? dfinal_states, bool silu, Tensor? seq_idx=None) -> "
        "(Tensor, Tensor, Tensor, Tensor)");
  m.def("causal_conv1d_update(Tensor x, Tensor(a!) conv_state, Tensor weight, Tensor? bias, "
        "bool silu, Tensor? cache_seqlens=None, Tensor? conv_state_indices=None) -> Tensor");
  m.def("selective_state_update(Tensor(a!) state, Tensor x, Tensor dt, Tensor A, Tensor B, "
        "Tensor C, Tensor? D, Tensor? z, Tensor? dt_bias, bool dt_softplus, "
        "Tensor? state_batch_indices=None) -> Tensor");
  m.def("mixer_step(Tensor hidden, Tensor? norm_weight, float eps, bool add_residual, bool residual_in_fp32, "
        "Tensor in_w, Tensor? in_b, Tensor conv_w, Tensor? conv_b, Tensor(a!) conv_state, Tensor x_w, "
        "Tensor dt_w, Tensor? dt_b, Tensor A, Tensor? D, Tensor(b!) ssm_state, Tensor out_w, "
        "Tensor? out_b) -> Tensor");
  m.def("norm_linear(Tensor hidden, Tensor? norm_weight, float eps, Tensor weight, Tensor? bias, "
        "bool out_float32) -> Tensor");
  m.def("mamba2_step(Tensor hidden, Tensor? norm_weight, float eps, bool add_residual, bool residual_in_fp32, "
        "Tensor in_w, Tensor? in_b, Tensor conv_w, Tensor? conv_b, Tensor(a!) conv_state, Tensor? dt_bias, "
        "Tensor A, Tensor? D, Tensor(b!) ssm_state, Tensor gate_norm_w, float gate_eps, Tensor out_w, "
        "Tensor? out_b) -> Tensor");
}

TORCH_LIBRARY_IMPL(mamba_cpu, CUDA, m) {
  using namespace mcpu_torch;
  m.impl("selective_scan_fwd", &selective_scan_fwd);
  m.impl("selective_scan_bwd", &selective_scan_bwd);
  m.impl("selective_scan_fwd_ckpt", &selective_scan_fwd_ckpt);
  m.impl("selective_scan_bwd_ckpt", &selective_scan_bwd_ckpt);
  m.impl("selective_scan_cfwd", &selective_scan_cfwd);
  m.impl("selective_scan_cbwd", &selective_scan_cbwd);
  m.impl("mamba_inner_fwd", &mamba_inner_fwd);
  m.impl("mamba_inner_bwd", &mamba_inner_bwd);
  m.impl("causal_conv1d_fwd", &causal_conv1d_fwd);
  m.impl("causal_conv1d_bwd", &causal_conv1d_bwd);
  m.impl("causal_conv1d_update", &causal_conv1d_update);
  m.impl("selective_state_update", &selective_state_update);
  m.impl("ssd_fwd", &ssd_fwd);
  m.impl("ssd_bwd", &ssd_bwd);
  m.impl("ssd_varlen_states", &ssd_varlen_states);
  m.impl("mixer_step", &mixer_step);
  m.impl("norm_linear", &norm_linear);
  m.impl("mamba2_step", &mamba2_step);
}

TORCH_LIBRARY_IMPL(mamba_cpu, Autograd, m) {
  using namespace mcpu_torch;
  m.impl("selective_scan_fwd", &selective_scan_fwd_autograd);
  m.impl("selective_scan_fwd_ckpt", &selective_scan_fwd_ckpt_autograd);
  m.impl("causal_conv1d_fwd", &causal_conv1d_fwd_autograd);
  // One decode step: no gradient flows through it.
  m.impl("mixer_step", torch::CppFunction::makeFallthrough());
  m.impl("norm_linear", torch::CppFunction::makeFallthrough());
  m.impl("mamba2_step", torch::CppFunction::makeFallthrough());
}

TORCH_LIBRARY_IMPL(mamba_cpu, ADInplaceOrView, m) {
  using namespace mcpu_torch;
  m.impl("causal_conv1d_update", &causal_conv1d_update_inplace);
  m.impl("selective_state_update", &selective_state_update_inplace);
  m.impl("mixer_step", &mixer_step_inplace);
  m.impl("mamba2_step", &mamba2_step_inplace);
}
