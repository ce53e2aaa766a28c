// torch operator library `cuda_transformer` on top of the C ABI.
//
// Same operator names, schemas, argument meaning and error messages as the reference's
// launchers (Transformer_launchers/*.cu registered through bindings.cpp:3-7).  Each op:
// validates its inputs with TORCH_CHECK (surfacing as a Python RuntimeError), allocates
// dense outputs on the input's device, and calls the gfx950 kernels through the C ABI on
// torch's current HIP stream.  Two schemas are added for LayerNorm, which the reference
// implements in plain torch only (gpt/gpt.py:47-59), and two for the fused linear+GELU products
// of the GPT MLP.
//
// This file is host-only C++; every kernel lives in libcuda_transformer_amd.so.
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cstdint>
#include <tuple>

#include "cuda_transformer_amd.h"

namespace cuda_transformer {
namespace {

// Largest dS workspace the flash_attention_bwd ops allocate, in bytes: by default 8 GiB of the
// MI355X's 288 GB; longer sequences run the stored-dS schedule in chunks of heads.  A cap below
// one head's dS tiles (0 in particular) selects the workspace-free recompute schedule.  Settable
// from Python with cuda_transformer_amd._C.set_bwd_workspace_cap(bytes).
constexpr int64_t kDefaultBwdWorkspaceCap = int64_t{8} << 30;
std::atomic<int64_t>& bwd_workspace_cap() {
  static std::atomic<int64_t> cap{kDefaultBwdWorkspaceCap};
  return cap;
}

// Workspace bytes the stored-dS schedule gets under the cap: whole heads only, and 0 (recompute)
// when not even one head's tiles fit.
int64_t capped_workspace(int64_t full, int64_t head) {
  const int64_t cap = bwd_workspace_cap().load();
  if (head <= 0 || cap < head) return 0;
  return std::min(full, cap / head * head);
}

void* stream_of(const at::Tensor& t) {
  return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

void check_rc(int rc) { TORCH_CHECK(rc == CTA_OK, cta_last_error()); }

// Which schedule the last flash_attention_bwd in this process ran: 1 stored dS, 0 recompute
// (no workspace: the faster 16-bit schedule, a cap below one head, or the allocator refused
// it), -1 none yet.  Process-wide, because autograd runs backward on its own device thread.
// Exposed to Python as cuda_transformer_amd._C.last_bwd_schedule().
std::atomic<int>& last_bwd_schedule() {
  static std::atomic<int> schedule{-1};
  return schedule;
}

void check_f32(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be a float32 tensor, got ",
              t.scalar_type());
}

template <size_t N>
std::array<int64_t, N> strides_of(const at::Tensor& t) {
  std::array<int64_t, N> s{};
  for (size_t d = 0; d < N; ++d) s[d] = t.size(d) == 1 ? 0 : t.stride(d);  // size-1 dims: unused
  return s;
}

// The attention kernels read 16-byte row segments: unit d-stride, strides divisible by 4,
// 16-byte aligned base, time stride in [0, 2^23).  Anything else is passed as a dense copy.
bool attn_layout_ok(const at::Tensor& t) {
  const auto s = strides_of<4>(t);
  return (t.size(3) == 1 || t.stride(3) == 1) && s[0] % 4 == 0 && s[1] % 4 == 0 &&
         s[2] % 4 == 0 && s[2] >= 0 && s[2] < ((int64_t)1 << 23) &&
         (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) == 0;
}

at::Tensor attn_operand(const at::Tensor& t) {
  if (attn_layout_ok(t)) return t;
  at::Tensor c = t.contiguous();
  if (!attn_layout_ok(c)) c = t.clone(at::MemoryFormat::Contiguous);
  return c;
}

at::Tensor dense(const at::Tensor& t) {
  at::Tensor c = t.contiguous();
  if ((reinterpret_cast<uintptr_t>(c.data_ptr()) & 15u) != 0) c = t.clone(at::MemoryFormat::Contiguous);
  return c;
}

// ------------------------------------------------------------------ linear layer
// cf. Transformer_launchers/linear_layer.cu:28-70
at::Tensor cuda_fma(at::Tensor x, at::Tensor weights, at::Tensor bias) {
  if (weights.dim() == 2) weights = weights.unsqueeze(0);
  TORCH_CHECK(x.dim() == 3, "x must be a 3D tensor (batch, m, k)");
  TORCH_CHECK(weights.dim() == 3, "weights must be a 2D or 3D tensor");
  TORCH_CHECK(bias.dim() == 1, "bias must be a 1D tensor");
  const int64_t x_batch = x.size(0), m = x.size(1), k = x.size(2), n = weights.size(2);
  TORCH_CHECK(weights.size(1) == k, "weights.size(1) must match x.size(2)");
  TORCH_CHECK(bias.size(0) == n, "bias.size(0) must match weights.size(2)");
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(weights.is_cuda(), "weights must be a CUDA tensor");
  TORCH_CHECK(bias.is_cuda(), "bias must be a CUDA tensor");
  check_f32(x, "x");
  check_f32(weights, "weights");
  check_f32(bias, "bias");
  TORCH_CHECK(weights.size(0) == 1 || weights.size(0) == x_batch,
              "weights.size(0) must be 1 or match x.size(0)");
  c10::OptionalDeviceGuard guard(x.device());
  at::Tensor out = at::empty({x_batch, m, n}, x.options());
  const auto xs = strides_of<3>(x);
  const auto ws = strides_of<3>(weights);
  const int64_t ws_bytes = cta_cuda_fma_workspace(x_batch, m, k, n);
  at::Tensor scratch;
  if (ws_bytes > 0) scratch = at::empty({ws_bytes / 4}, x.options());
  check_rc(cta_cuda_fma(x.data_ptr<float>(), xs.data(), weights.data_ptr<float>(), ws.data(),
                        bias.data_ptr<float>(), bias.stride(0), x_batch, m, k, n,
                        weights.size(0), out.data_ptr<float>(),
                        ws_bytes > 0 ? scratch.data_ptr<float>() : nullptr, stream_of(x)));
  return out;
}

// Shared checks of the fused linear+GELU ops: x (batch, m, k), weights (k, n) or (1|batch, k, n),
// same messages as cuda_fma.  Returns weights as 3-D.
at::Tensor check_linear(const at::Tensor& x, at::Tensor weights) {
  if (weights.dim() == 2) weights = weights.unsqueeze(0);
  TORCH_CHECK(x.dim() == 3, "x must be a 3D tensor (batch, m, k)");
  TORCH_CHECK(weights.dim() == 3, "weights must be a 2D or 3D tensor");
  TORCH_CHECK(weights.size(1) == x.size(2), "weights.size(1) must match x.size(2)");
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(weights.is_cuda(), "weights must be a CUDA tensor");
  check_f32(x, "x");
  check_f32(weights, "weights");
  TORCH_CHECK(weights.size(0) == 1 || weights.size(0) == x.size(0),
              "weights.size(0) must be 1 or match x.size(0)");
  return weights;
}

// (pre, out) = (x W + b, GELU(x W + b)) from one GEMM whose epilogue writes both.  New op: the
// GPT MLP's fc1 -> GELU (gpt/gpt.py:134-135) without the second pass over pre.
// deriv_form: the first output is GELU'(x W + b) (cta_cuda_fma_gelu_deriv) instead of pre.
std::tuple<at::Tensor, at::Tensor> fma_gelu_impl(at::Tensor x, at::Tensor weights,
                                                 at::Tensor bias, bool tanh_form,
                                                 bool deriv_form = false) {
  weights = check_linear(x, weights);
  TORCH_CHECK(bias.dim() == 1, "bias must be a 1D tensor");
  TORCH_CHECK(bias.size(0) == weights.size(2), "bias.size(0) must match weights.size(2)");
  TORCH_CHECK(bias.is_cuda(), "bias must be a CUDA tensor");
  check_f32(bias, "bias");
  const int64_t batch = x.size(0), m = x.size(1), k = x.size(2), n = weights.size(2);
  c10::OptionalDeviceGuard guard(x.device());
  at::Tensor pre = at::empty({batch, m, n}, x.options());
  at::Tensor out = at::empty({batch, m, n}, x.options());
  const auto xs = strides_of<3>(x);
  const auto wst = strides_of<3>(weights);
  const int64_t ws_bytes = cta_cuda_fma_workspace(batch, m, k, n);
  at::Tensor scratch;
  if (ws_bytes > 0) scratch = at::empty({ws_bytes / 4}, x.options());
  const auto fn = deriv_form ? (tanh_form ? cta_cuda_fma_gelu_tanh_deriv : cta_cuda_fma_gelu_deriv)
                             : (tanh_form ? cta_cuda_fma_gelu_tanh : cta_cuda_fma_gelu);
  check_rc(fn(x.data_ptr<float>(), xs.data(), weights.data_ptr<float>(),
                             wst.data(), bias.data_ptr<float>(), bias.stride(0), batch, m, k, n,
                             weights.size(0), pre.data_ptr<float>(), out.data_ptr<float>(),
                             ws_bytes > 0 ? scratch.data_ptr<float>() : nullptr, stream_of(x)));
  return {pre, out};
}

// dx = (dy W) * GELU'(pre).  New op: CudaLinearLayer.backward's dx product of fc2 followed by
// CudaGeluLayer.backward (cuda_linear_layer.py:19-23, cuda_gelu_layer.py:12-14) in one pass.
// mul_form: pre holds a saved GELU'(pre) and dx = (dy W) * pre (cta_cuda_fma_mul).
at::Tensor fma_gelu_grad_impl(at::Tensor dy, at::Tensor weights, at::Tensor pre,
                              bool tanh_form, bool mul_form = false) {
  weights = check_linear(dy, weights);
  const int64_t batch = dy.size(0), m = dy.size(1), k = dy.size(2), n = weights.size(2);
  const char* name = mul_form ? "d" : "pre";
  TORCH_CHECK(pre.dim() == 3 && pre.size(0) == batch && pre.size(1) == m && pre.size(2) == n,
              name, " must have shape (dy.size(0), dy.size(1), weights.size(-1))");
  TORCH_CHECK(pre.is_cuda(), name, " must be a CUDA tensor");
  check_f32(pre, name);
  c10::OptionalDeviceGuard guard(dy.device());
  const at::Tensor pd = pre.contiguous();
  at::Tensor dx = at::empty({batch, m, n}, dy.options());
  const auto ds = strides_of<3>(dy);
  const auto wst = strides_of<3>(weights);
  const int64_t ws_bytes = cta_cuda_fma_workspace(batch, m, k, n);
  at::Tensor scratch;
  if (ws_bytes > 0) scratch = at::empty({ws_bytes / 4}, dy.options());
  const auto fn = mul_form ? cta_cuda_fma_mul
                           : (tanh_form ? cta_cuda_fma_gelu_tanh_grad : cta_cuda_fma_gelu_grad);
  check_rc(fn(dy.data_ptr<float>(), ds.data(), weights.data_ptr<float>(),
                                  wst.data(), pd.data_ptr<float>(), batch, m, k, n,
                                  weights.size(0), dx.data_ptr<float>(),
                                  ws_bytes > 0 ? scratch.data_ptr<float>() : nullptr,
                                  stream_of(dy)));
  return dx;
}

std::tuple<at::Tensor, at::Tensor> cuda_fma_gelu(at::Tensor x, at::Tensor weights,
                                                 at::Tensor bias) {
  return fma_gelu_impl(x, weights, bias, false);
}
at::Tensor cuda_fma_gelu_grad(at::Tensor dy, at::Tensor weights, at::Tensor pre) {
  return fma_gelu_grad_impl(dy, weights, pre, false);
}
// The same two products with the tanh-approximated GELU (new ops, no reference counterpart).
std::tuple<at::Tensor, at::Tensor> cuda_fma_gelu_tanh(at::Tensor x, at::Tensor weights,
                                                      at::Tensor bias) {
  return fma_gelu_impl(x, weights, bias, true);
}
at::Tensor cuda_fma_gelu_tanh_grad(at::Tensor dy, at::Tensor weights, at::Tensor pre) {
  return fma_gelu_grad_impl(dy, weights, pre, true);
}
// (GELU'(x W + b), GELU(x W + b)) and its backward (dy W) * d: the derivative is evaluated in
// the forward epilogue, which already has the normal CDF (new ops, no reference counterpart).
std::tuple<at::Tensor, at::Tensor> cuda_fma_gelu_deriv(at::Tensor x, at::Tensor weights,
                                                       at::Tensor bias) {
  return fma_gelu_impl(x, weights, bias, false, true);
}
std::tuple<at::Tensor, at::Tensor> cuda_fma_gelu_tanh_deriv(at::Tensor x, at::Tensor weights,
                                                            at::Tensor bias) {
  return fma_gelu_impl(x, weights, bias, true, true);
}
at::Tensor cuda_fma_mul(at::Tensor dy, at::Tensor weights, at::Tensor d) {
  return fma_gelu_grad_impl(dy, weights, d, false, true);
}

// cf. linear_layer.cu:74-97
at::Tensor db_calculation(at::Tensor dy) {
  TORCH_CHECK(dy.dim() == 3, "dy must be a 3D tensor (batch, m, n)");
  TORCH_CHECK(dy.is_cuda(), "dy must be a CUDA tensor");
  check_f32(dy, "dy");
  const int64_t batch = dy.size(0), m = dy.size(1), n = dy.size(2);
  c10::OptionalDeviceGuard guard(dy.device());
  at::Tensor db = at::empty({n}, dy.options());
  const int64_t ws_bytes = cta_db_calculation_workspace(batch, m, n);
  at::Tensor ws = at::empty({std::max<int64_t>(1, ws_bytes / 4)}, dy.options());
  const auto s = strides_of<3>(dy);
  check_rc(cta_db_calculation(dy.data_ptr<float>(), s.data(), batch, m, n, db.data_ptr<float>(),
                              ws.data_ptr<float>(), stream_of(dy)));
  return db;
}

// (dW, db) = (x^T dy, column sums of dy) over the rows of x (..., k) and dy (..., n), leading
// dims folded into the rows: CudaLinearLayer.backward's weight product and db_calculation
// (cuda_linear_layer.py:21-27) in one GEMM that sums dy's columns as it streams them.
std::tuple<at::Tensor, at::Tensor> linear_weight_bias_grad(at::Tensor x, at::Tensor dy) {
  TORCH_CHECK(x.dim() >= 1 && dy.dim() == x.dim(), "x and dy must have the same rank");
  TORCH_CHECK(x.sizes().slice(0, x.dim() - 1) == dy.sizes().slice(0, dy.dim() - 1),
              "x and dy must agree in every dim but the last");
  TORCH_CHECK(x.is_cuda() && dy.is_cuda(), "x and dy must be CUDA tensors");
  check_f32(x, "x");
  check_f32(dy, "dy");
  const int64_t k = x.size(-1), n = dy.size(-1);
  int64_t rows = 1;
  for (int64_t d = 0; d + 1 < x.dim(); ++d) rows *= x.size(d);
  const at::Tensor x2 = x.reshape({rows, k});
  const at::Tensor d2 = dy.reshape({rows, n});
  c10::OptionalDeviceGuard guard(x.device());
  at::Tensor dw = at::empty({k, n}, x.options());
  at::Tensor db = at::empty({n}, x.options());
  const int64_t ws_bytes = cta_linear_weight_bias_grad_workspace(rows, k, n);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({ws_bytes / 4}, x.options());
  const int64_t xs[2] = {x2.stride(0), x2.stride(1)};
  const int64_t ds[2] = {d2.stride(0), d2.stride(1)};
  check_rc(cta_linear_weight_bias_grad(x2.data_ptr<float>(), xs, d2.data_ptr<float>(), ds, rows,
                                       k, n, dw.data_ptr<float>(), db.data_ptr<float>(),
                                       ws_bytes > 0 ? ws.data_ptr<float>() : nullptr,
                                       stream_of(x)));
  return {dw, db};
}

// ------------------------------------------------------------------ GELU
// cf. Transformer_launchers/gelu_activation.cu:22-77
at::Tensor gelu_activation(at::Tensor x) {
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
  check_f32(x, "x");
  c10::OptionalDeviceGuard guard(x.device());
  const at::Tensor xd = dense(x);
  at::Tensor out = at::empty(x.sizes(), x.options());
  check_rc(cta_gelu_fwd(xd.data_ptr<float>(), out.data_ptr<float>(), x.numel(), stream_of(x)));
  return out;
}

at::Tensor gelu_activation_bwd(at::Tensor x, at::Tensor dy) {
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
  TORCH_CHECK(dy.is_cuda(), "dy must be a CUDA tensor");
  TORCH_CHECK(dy.is_contiguous(), "dy must be contiguous");
  check_f32(x, "x");
  check_f32(dy, "dy");
  TORCH_CHECK(x.numel() == dy.numel(), "x and dy must have the same number of elements");
  c10::OptionalDeviceGuard guard(x.device());
  const at::Tensor xd = dense(x), gd = dense(dy);
  at::Tensor out = at::empty(x.sizes(), x.options());
  check_rc(cta_gelu_bwd(xd.data_ptr<float>(), gd.data_ptr<float>(), out.data_ptr<float>(),
                        x.numel(), stream_of(x)));
  return out;
}

// ------------------------------------------------------------------ tanh GELU
// New ops with no reference launcher: F.gelu(x, approximate="tanh") and its input gradient,
// with the same checks and layout as gelu_activation / gelu_activation_bwd above.
at::Tensor gelu_tanh_activation(at::Tensor x) {
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
  check_f32(x, "x");
  c10::OptionalDeviceGuard guard(x.device());
  const at::Tensor xd = dense(x);
  at::Tensor out = at::empty(x.sizes(), x.options());
  check_rc(cta_gelu_tanh_fwd(xd.data_ptr<float>(), out.data_ptr<float>(), x.numel(),
                             stream_of(x)));
  return out;
}

at::Tensor gelu_tanh_activation_bwd(at::Tensor x, at::Tensor dy) {
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
  TORCH_CHECK(dy.is_cuda(), "dy must be a CUDA tensor");
  TORCH_CHECK(dy.is_contiguous(), "dy must be contiguous");
  check_f32(x, "x");
  check_f32(dy, "dy");
  TORCH_CHECK(x.numel() == dy.numel(), "x and dy must have the same number of elements");
  c10::OptionalDeviceGuard guard(x.device());
  const at::Tensor xd = dense(x), gd = dense(dy);
  at::Tensor out = at::empty(x.sizes(), x.options());
  check_rc(cta_gelu_tanh_bwd(xd.data_ptr<float>(), gd.data_ptr<float>(), out.data_ptr<float>(),
                             x.numel(), stream_of(x)));
  return out;
}

// ------------------------------------------------------------------ softmax
// cf. Transformer_launchers/softmax_layer.cu:22-78
at::Tensor cuda_softmax(at::Tensor x) {
  TORCH_CHECK(x.dim() == 3, "x must be a 3D tensor");
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
  check_f32(x, "x");
  c10::OptionalDeviceGuard guard(x.device());
  const at::Tensor xd = dense(x);
  at::Tensor out = at::empty(x.sizes(), x.options());
  check_rc(cta_softmax_fwd(xd.data_ptr<float>(), out.data_ptr<float>(), x.size(0) * x.size(1),
                           x.size(2), stream_of(x)));
  return out;
}

at::Tensor cuda_softmax_bwd(at::Tensor probs, at::Tensor dp) {
  TORCH_CHECK(probs.dim() == 3, "probs must be a 3D tensor");
  TORCH_CHECK(probs.is_cuda(), "probs must be a CUDA tensor");
  TORCH_CHECK(probs.is_contiguous(), "probs must be contiguous");
  TORCH_CHECK(dp.dim() == 3, "dp must be a 3D tensor");
  TORCH_CHECK(dp.is_cuda(), "dp must be a CUDA tensor");
  TORCH_CHECK(dp.is_contiguous(), "dp must be contiguous");
  check_f32(probs, "probs");
  check_f32(dp, "dp");
  TORCH_CHECK(probs.sizes() == dp.sizes(), "probs and dp must have the same shape");
  c10::OptionalDeviceGuard guard(probs.device());
  const at::Tensor pd = dense(probs), gd = dense(dp);
  at::Tensor out = at::empty(probs.sizes(), probs.options());
  check_rc(cta_softmax_bwd(pd.data_ptr<float>(), gd.data_ptr<float>(), out.data_ptr<float>(),
                           probs.size(0) * probs.size(1), probs.size(2), stream_of(probs)));
  return out;
}

// ------------------------------------------------------------------ LayerNorm (new)
// LayerNorm over the last dim of x, or of xsum = x + f (returned first) when f is given.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> layernorm_fwd_impl(
    const at::Tensor& x, const c10::optional<at::Tensor>& f, const at::Tensor& gamma,
    const at::Tensor& beta, double eps) {
  TORCH_CHECK(x.dim() >= 1, "x must have at least one dimension");
  TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
  TORCH_CHECK(gamma.is_cuda(), "gamma must be a CUDA tensor");
  TORCH_CHECK(beta.is_cuda(), "beta must be a CUDA tensor");
  check_f32(x, "x");
  check_f32(gamma, "gamma");
  check_f32(beta, "beta");
  if (f) {
    TORCH_CHECK(f->is_cuda(), "f must be a CUDA tensor");
    check_f32(*f, "f");
    TORCH_CHECK(f->sizes() == x.sizes(), "f must have the shape of x");
  }
  const int64_t n = x.size(-1);
  TORCH_CHECK(gamma.numel() == n && beta.numel() == n,
              "gamma and beta must have x.size(-1) elements");
  c10::OptionalDeviceGuard guard(x.device());
  const at::Tensor xd = dense(x), gd = dense(gamma), bd = dense(beta);
  const at::Tensor fd = f ? dense(*f) : at::Tensor();
  const int64_t rows = n == 0 ? 0 : x.numel() / n;
  at::Tensor y = at::empty(x.sizes(), x.options());
  at::Tensor xsum = f ? at::empty(x.sizes(), x.options()) : at::Tensor();
  auto stat_shape = x.sizes().vec();
  stat_shape.pop_back();
  at::Tensor mean = at::empty(stat_shape, x.options());
  at::Tensor rstd = at::empty(stat_shape, x.options());
  if (f)
    check_rc(cta_add_layernorm_fwd(xd.data_ptr<float>(), fd.data_ptr<float>(),
                                   gd.data_ptr<float>(), bd.data_ptr<float>(), rows, n,
                                   static_cast<float>(eps), xsum.data_ptr<float>(),
                                   y.data_ptr<float>(), mean.data_ptr<float>(),
                                   rstd.data_ptr<float>(), stream_of(x)));
  else
    check_rc(cta_layernorm_fwd(xd.data_ptr<float>(), gd.data_ptr<float>(), bd.data_ptr<float>(),
                               rows, n, static_cast<float>(eps), y.data_ptr<float>(),
                               mean.data_ptr<float>(), rstd.data_ptr<float>(), stream_of(x)));
  return {xsum, y, mean, rstd};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> layernorm_fwd(at::Tensor x, at::Tensor gamma,
                                                             at::Tensor beta, double eps) {
  auto r = layernorm_fwd_impl(x, c10::nullopt, gamma, beta, eps);
  return {std::get<1>(r), std::get<2>(r), std::get<3>(r)};
}

// xsum = x + f and LayerNorm(xsum) in one pass.  New op: a pre-LN block's residual add and the
// LayerNorm after it (gpt/gpt.py:147-150).
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> add_layernorm_fwd(
    at::Tensor x, at::Tensor f, at::Tensor gamma, at::Tensor beta, double eps) {
  return layernorm_fwd_impl(x, f, gamma, beta, eps);
}

// LayerNorm backward at x; with dres, dx also receives dres.
std::tuple<at::Tensor, at::Tensor, at::Tensor> layernorm_bwd_impl(
    const at::Tensor& x, const at::Tensor& gamma, const at::Tensor& mean, const at::Tensor& rstd,
    const at::Tensor& dy, const c10::optional<at::Tensor>& dres) {
  TORCH_CHECK(x.is_cuda() && gamma.is_cuda() && mean.is_cuda() && rstd.is_cuda() && dy.is_cuda(),
              "layernorm_bwd inputs must be CUDA tensors");
  check_f32(x, "x");
  check_f32(gamma, "gamma");
  check_f32(mean, "mean");
  check_f32(rstd, "rstd");
  check_f32(dy, "dy");
  if (dres) {
    TORCH_CHECK(dres->is_cuda(), "dres must be a CUDA tensor");
    check_f32(*dres, "dres");
    TORCH_CHECK(dres->sizes() == x.sizes(), "dres must have the shape of x");
  }
  const int64_t n = x.size(-1);
  TORCH_CHECK(dy.sizes() == x.sizes(), "dy must have the shape of x");
  TORCH_CHECK(gamma.numel() == n, "gamma must have x.size(-1) elements");
  const int64_t rows = n == 0 ? 0 : x.numel() / n;
  TORCH_CHECK(mean.numel() == rows && rstd.numel() == rows, "mean/rstd must have one value per row");
  c10::OptionalDeviceGuard guard(x.device());
  const at::Tensor xd = dense(x), gd = dense(gamma), md = dense(mean), rd = dense(rstd),
                   dd = dense(dy);
  const at::Tensor rsd = dres ? dense(*dres) : at::Tensor();
  at::Tensor dx = at::empty(x.sizes(), x.options());
  at::Tensor dgamma = at::empty({n}, x.options());
  at::Tensor dbeta = at::empty({n}, x.options());
  const int64_t ws_bytes = cta_layernorm_bwd_workspace(rows, n);
  at::Tensor ws = at::empty({std::max<int64_t>(1, ws_bytes / 4)}, x.options());
  if (dres)
    check_rc(cta_add_layernorm_bwd(xd.data_ptr<float>(), gd.data_ptr<float>(),
                                   md.data_ptr<float>(), rd.data_ptr<float>(),
                                   dd.data_ptr<float>(), rsd.data_ptr<float>(), rows, n,
                                   dx.data_ptr<float>(), dgamma.data_ptr<float>(),
                                   dbeta.data_ptr<float>(), ws.data_ptr<float>(), stream_of(x)));
  else
    check_rc(cta_layernorm_bwd(xd.data_ptr<float>(), gd.data_ptr<float>(), md.data_ptr<float>(),
                               rd.data_ptr<float>(), dd.data_ptr<float>(), rows, n,
                               dx.data_ptr<float>(), dgamma.data_ptr<float>(),
                               dbeta.data_ptr<float>(), ws.data_ptr<float>(), stream_of(x)));
  return {dx, dgamma, dbeta};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> layernorm_bwd(at::Tensor x, at::Tensor gamma,
                                                             at::Tensor mean, at::Tensor rstd,
                                                             at::Tensor dy) {
  return layernorm_bwd_impl(x, gamma, mean, rstd, dy, c10::nullopt);
}

// Backward of add_layernorm_fwd: (LayerNorm backward of dy at xsum) + dres, dgamma, dbeta.
std::tuple<at::Tensor, at::Tensor, at::Tensor> add_layernorm_bwd(at::Tensor xsum,
                                                                 at::Tensor gamma,
                                                                 at::Tensor mean, at::Tensor rstd,
                                                                 at::Tensor dy, at::Tensor dres) {
  return layernorm_bwd_impl(xsum, gamma, mean, rstd, dy, dres);
}

// ------------------------------------------------------------------ naive attention
// cf. Transformer_launchers/causal_self_attn_layer.cu:24-67
std::tuple<at::Tensor, at::Tensor> causal_self_attention_fwd(at::Tensor qkv, int64_t nh,
                                                             bool causal) {
  TORCH_CHECK(qkv.dim() == 3, "qkv must be a 3D tensor (B, T, 3C)");
  TORCH_CHECK(qkv.is_cuda(), "qkv must be a CUDA tensor");
  TORCH_CHECK(qkv.is_contiguous(), "qkv must be contiguous");
  check_f32(qkv, "qkv");
  const int64_t B = qkv.size(0), T = qkv.size(1), C = qkv.size(2) / 3;
  TORCH_CHECK(nh > 0 && C % nh == 0, "C must be divisible by nh");
  c10::OptionalDeviceGuard guard(qkv.device());
  const at::Tensor qd = dense(qkv);
  at::Tensor s = at::empty({B, nh, T, T}, qkv.options());
  at::Tensor out = at::empty({B, T, C}, qkv.options());
  check_rc(cta_causal_self_attention_fwd(qd.data_ptr<float>(), B, T, C, nh, causal ? 1 : 0,
                                         out.data_ptr<float>(), s.data_ptr<float>(),
                                         stream_of(qkv)));
  return {out, s};
}

// cf. causal_self_attn_layer.cu:70-132; inputs (B*nh, T, hs), probs (B*nh, T, T)
std::tuple<at::Tensor, at::Tensor, at::Tensor> causal_self_attention_bwd(
    at::Tensor Q, at::Tensor K, at::Tensor V, at::Tensor probs, at::Tensor dO) {
  TORCH_CHECK(Q.is_cuda(), "q must be a CUDA tensor");
  TORCH_CHECK(K.is_cuda(), "k must be a CUDA tensor");
  TORCH_CHECK(V.is_cuda(), "v must be a CUDA tensor");
  TORCH_CHECK(probs.is_cuda(), "probs must be a CUDA tensor");
  TORCH_CHECK(dO.is_cuda(), "dO must be a CUDA tensor");
  for (const auto* t : {&Q, &K, &V, &probs, &dO}) check_f32(*t, "input");
  TORCH_CHECK(Q.dim() == 3, "Q must be (B*nh, T, hs)");
  const int64_t BH = Q.size(0), T = Q.size(1), hs = Q.size(2);
  TORCH_CHECK(K.sizes() == Q.sizes() && V.sizes() == Q.sizes() && dO.sizes() == Q.sizes(),
              "Q, K, V and dO must have the same shape");
  TORCH_CHECK(probs.dim() == 3 && probs.size(0) == BH && probs.size(1) == T && probs.size(2) == T,
              "probs must be (B*nh, T, T)");
  c10::OptionalDeviceGuard guard(Q.device());
  const at::Tensor pd = dense(probs);
  at::Tensor dq = at::empty({BH, T, hs}, Q.options());
  at::Tensor dk = at::empty({BH, T, hs}, Q.options());
  at::Tensor dv = at::empty({BH, T, hs}, Q.options());
  const int64_t ws_bytes = cta_causal_self_attention_bwd_workspace(BH, T);
  at::Tensor ws = at::empty({std::max<int64_t>(1, ws_bytes / 4)}, Q.options());
  const auto qs = strides_of<3>(Q), ks = strides_of<3>(K), vs = strides_of<3>(V),
             gs = strides_of<3>(dO);
  check_rc(cta_causal_self_attention_bwd(
      Q.data_ptr<float>(), qs.data(), K.data_ptr<float>(), ks.data(), V.data_ptr<float>(),
      vs.data(), pd.data_ptr<float>(), dO.data_ptr<float>(), gs.data(), BH, T, hs,
      dq.data_ptr<float>(), dk.data_ptr<float>(), dv.data_ptr<float>(), ws.data_ptr<float>(),
      stream_of(Q)));
  return {dq, dk, dv};
}

// ------------------------------------------------------------------ FlashAttention-2
// 16-bit inputs, bfloat16 or float16 (an extension: the reference's kernels are FP32 only):
// O in the input type, L in FP32.
bool is_half16(const at::Tensor& t) {
  return t.scalar_type() == at::kBFloat16 || t.scalar_type() == at::kHalf;
}

bool attn_layout_half_ok(const at::Tensor& t) {
  const auto s = strides_of<4>(t);
  return (t.size(3) == 1 || t.stride(3) == 1) && s[0] % 8 == 0 && s[1] % 8 == 0 &&
         s[2] % 8 == 0 && s[2] >= 0 && s[2] < ((int64_t)1 << 24) &&
         (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) == 0;
}

at::Tensor attn_operand_half(const at::Tensor& t) {
  if (attn_layout_half_ok(t)) return t;
  at::Tensor c = t.contiguous();
  if (!attn_layout_half_ok(c)) c = t.clone(at::MemoryFormat::Contiguous);
  return c;
}

std::tuple<at::Tensor, at::Tensor> flash_attention_fwd_half(const at::Tensor& Q,
                                                            const at::Tensor& K,
                                                            const at::Tensor& V, bool causal) {
  const int64_t B = Q.size(0), nh = Q.size(1), T = Q.size(2), hs = Q.size(3);
  const bool bf = Q.scalar_type() == at::kBFloat16;
  TORCH_CHECK(K.scalar_type() == Q.scalar_type() && V.scalar_type() == Q.scalar_type(),
              "Q, K and V must have the same dtype (float32, bfloat16 or float16)");
  TORCH_CHECK(hs == 32 || hs == 64 || hs == 128,
              "Unsupported head dimension! Only hs=32, hs=64, and hs=128 are supported.");
  c10::OptionalDeviceGuard guard(Q.device());
  at::Tensor O = at::empty({B, nh, T, hs}, Q.options());
  at::Tensor L = at::empty({B, nh, T}, Q.options().dtype(at::kFloat));
  const at::Tensor q = attn_operand_half(Q), k = attn_operand_half(K), v = attn_operand_half(V);
  const auto qs = strides_of<4>(q), ks = strides_of<4>(k), vs = strides_of<4>(v);
  check_rc((bf ? cta_flash_attention_fwd_bf16 : cta_flash_attention_fwd_f16)(
      reinterpret_cast<const uint16_t*>(q.data_ptr()), qs.data(),
      reinterpret_cast<const uint16_t*>(k.data_ptr()), ks.data(),
      reinterpret_cast<const uint16_t*>(v.data_ptr()), vs.data(), B, nh, T, hs, causal ? 1 : 0,
      reinterpret_cast<uint16_t*>(O.data_ptr()), L.data_ptr<float>(), stream_of(Q)));
  return {O, L};
}

// Scratch with which the FP32 forward splits a small grid's work over two or three times the
// workgroups (cta_flash_attention_fwd_workspace; none for grids that fill the GPU).  If the allocator
// cannot supply it, the forward runs unsplit (ws_bytes = 0): same results to rounding.
at::Tensor fwd_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs, bool causal,
                         const at::TensorOptions& opts, int64_t& ws_bytes) {
  ws_bytes = cta_flash_attention_fwd_workspace(B, nh, T, hs, causal ? 1 : 0);
  at::Tensor ws;
  if (ws_bytes > 0) {
    try {
      ws = at::empty({ws_bytes / static_cast<int64_t>(sizeof(float))}, opts);
    } catch (const c10::OutOfMemoryError&) {
      ws_bytes = 0;
    }
  }
  return ws;
}

// cf. Transformer_launchers/flash_attn_launcher.cu:22-65
std::tuple<at::Tensor, at::Tensor> flash_attention_fwd(at::Tensor Q, at::Tensor K, at::Tensor V,
                                                       bool causal) {
  TORCH_CHECK(Q.dim() == 4, "Q must be a 4D tensor (B, nh, T, hs)");
  const int64_t B = Q.size(0), nh = Q.size(1), T = Q.size(2), hs = Q.size(3);
  TORCH_CHECK(Q.is_cuda(), "Q must be a CUDA tensor");
  TORCH_CHECK(K.is_cuda(), "K must be a CUDA tensor");
  TORCH_CHECK(V.is_cuda(), "V must be a CUDA tensor");
  TORCH_CHECK(K.sizes() == Q.sizes() && V.sizes() == Q.sizes(), "Q, K and V must have the same shape");
  if (is_half16(Q)) return flash_attention_fwd_half(Q, K, V, causal);
  check_f32(Q, "Q");
  check_f32(K, "K");
  check_f32(V, "V");
  c10::OptionalDeviceGuard guard(Q.device());
  at::Tensor O = at::empty({B, nh, T, hs}, Q.options());
  at::Tensor L = at::empty({B, nh, T}, Q.options());
  if (hs != 32 && hs != 64 && hs != 128)
    TORCH_CHECK(false, "Unsupported head dimension! Only hs=32, hs=64, and hs=128 are supported.");
  const at::Tensor q = attn_operand(Q), k = attn_operand(K), v = attn_operand(V);
  const auto qs = strides_of<4>(q), ks = strides_of<4>(k), vs = strides_of<4>(v);
  const int64_t os[4] = {nh * T * hs, T * hs, hs, 1};
  int64_t ws_bytes = 0;
  const at::Tensor ws = fwd_workspace(B, nh, T, hs, causal, Q.options(), ws_bytes);
  check_rc(cta_flash_attention_fwd_ex(q.data_ptr<float>(), qs.data(), k.data_ptr<float>(),
                                      ks.data(), v.data_ptr<float>(), vs.data(), B, nh, T, hs,
                                      causal ? 1 : 0, O.data_ptr<float>(), os, L.data_ptr<float>(),
                                      ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
                                      stream_of(Q)));
  return {O, L};
}

// Workspace for the stored-dS schedule of the FP32 backward: every head's dS tiles up to the
// workspace cap (chunked over heads beyond that).  If the cap holds less than one head, or the
// allocator cannot supply it, the kernels run the recompute schedule, which needs no workspace
// (ws_bytes = 0).
at::Tensor bwd_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs, bool causal,
                         const at::TensorOptions& opts, int64_t& ws_bytes) {
  const int64_t full = cta_flash_attention_bwd_workspace(B, nh, T, hs, causal ? 1 : 0);
  ws_bytes = capped_workspace(full, cta_flash_attention_bwd_workspace(1, 1, T, hs, causal ? 1 : 0));
  // every head's dS tiles fit: room for a small grid's split dK/dV and dQ-from-dS stages too
  if (ws_bytes == full && full > 0)
    ws_bytes += cta_flash_attention_bwd_split_workspace(B, nh, T, hs, causal ? 1 : 0);
  at::Tensor ws;
  if (ws_bytes > 0) {
    try {
      ws = at::empty({ws_bytes / static_cast<int64_t>(sizeof(float))}, opts);
    } catch (const c10::OutOfMemoryError&) {
      ws_bytes = 0;
      TORCH_WARN_ONCE(
          "flash_attention_bwd: the dS workspace could not be allocated; running the "
          "recompute schedule (dQ recomputes S and dP, about 20% slower, same results to "
          "rounding)");
    }
  }
  last_bwd_schedule().store(ws_bytes > 0 ? 1 : 0);
  return ws;
}

// 16-bit backward (extension): the FP32 op's two schedules, the stored one with a 16-bit dS
// workspace from torch's caching allocator under the same cap (chunked over heads beyond it).
std::tuple<at::Tensor, at::Tensor, at::Tensor> flash_attention_bwd_half(
    const at::Tensor& Q, const at::Tensor& K, const at::Tensor& V, const at::Tensor& O,
    const at::Tensor& dO, const at::Tensor& L, bool causal) {
  const int64_t B = Q.size(0), nh = Q.size(1), T = Q.size(2), hs = Q.size(3);
  const bool bf = Q.scalar_type() == at::kBFloat16;
  for (const auto* t : {&K, &V, &O, &dO})
    TORCH_CHECK(t->scalar_type() == Q.scalar_type(),
                "Q, K, V, O and dO must have the same dtype (float32, bfloat16 or float16)");
  TORCH_CHECK(L.scalar_type() == at::kFloat, "L must be a float32 tensor");
  TORCH_CHECK(K.sizes() == Q.sizes() && V.sizes() == Q.sizes() && O.sizes() == Q.sizes() &&
                  dO.sizes() == Q.sizes(),
              "Q, K, V, O and dO must have the same shape");
  TORCH_CHECK(L.dim() == 3 && L.size(0) == B && L.size(1) == nh && L.size(2) == T,
              "L must have shape (B, nh, T)");
  TORCH_CHECK(hs == 32 || hs == 64 || hs == 128,
              "Unsupported head dimension! Only hs=32, hs=64, and hs=128 are supported.");
  c10::OptionalDeviceGuard guard(Q.device());
  at::Tensor dQ = at::empty({B, nh, T, hs}, Q.options());
  at::Tensor dK = at::empty({B, nh, T, hs}, Q.options());
  at::Tensor dV = at::empty({B, nh, T, hs}, Q.options());
  if (B * nh * T == 0) return {dQ, dK, dV};
  at::Tensor delta = at::empty({B, nh, T}, Q.options().dtype(at::kFloat));
  // In 16 bits the workspace-free recompute schedule is the faster one at hs = 32 and 64
  // (measured at B4 H32 N4096: causal hs 64 1.15 against 1.49 ms, hs 32 0.71 against 1.28 ms;
  // B1 H16 N16384 and B4 H4 N4096 likewise), where its dQ kernel holds two waves per SIMD; at
  // hs = 128 it holds one and the stored-dS schedule is faster (2.49 against 3.39 ms causal).
  // So hs = 128 takes the stored schedule when the cap holds at least one head's 16-bit dS
  // tiles and the allocator supplies them; everything else recomputes.
  int64_t ws_bytes =
      hs == 128
          ? capped_workspace(cta_flash_attention_bwd_bf16_workspace(B, nh, T, hs, causal ? 1 : 0),
                             cta_flash_attention_bwd_bf16_workspace(1, 1, T, hs, causal ? 1 : 0))
          : 0;
  at::Tensor ws;
  if (ws_bytes > 0) {
    try {
      ws = at::empty({(ws_bytes + 15) / 16 * 4}, Q.options().dtype(at::kFloat));
    } catch (const c10::OutOfMemoryError&) {
      ws_bytes = 0;
      TORCH_WARN_ONCE(
          "flash_attention_bwd (16-bit): the dS workspace could not be allocated; running the "
          "recompute schedule (dQ recomputes S and dP, same results to rounding)");
    }
  }
  last_bwd_schedule().store(ws_bytes > 0 ? 1 : 0);
  const at::Tensor q = attn_operand_half(Q), k = attn_operand_half(K), v = attn_operand_half(V),
                   o = attn_operand_half(O), g = attn_operand_half(dO);
  const auto qs = strides_of<4>(q), ks = strides_of<4>(k), vs = strides_of<4>(v),
             os = strides_of<4>(o), gs = strides_of<4>(g);
  const auto ls = strides_of<3>(L);
  auto u16 = [](const at::Tensor& t) { return reinterpret_cast<const uint16_t*>(t.data_ptr()); };
  auto w16 = [](at::Tensor& t) { return reinterpret_cast<uint16_t*>(t.data_ptr()); };
  check_rc((bf ? cta_flash_attention_bwd_bf16 : cta_flash_attention_bwd_f16)(u16(q), qs.data(), u16(k), ks.data(), u16(v), vs.data(),
                                        u16(o), os.data(), u16(g), gs.data(),
                                        L.data_ptr<float>(), ls.data(), B, nh, T, hs,
                                        causal ? 1 : 0, w16(dQ), w16(dK), w16(dV),
                                        delta.data_ptr<float>(),
                                        ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes,
                                        stream_of(Q)));
  return {dQ, dK, dV};
}

// cf. flash_attn_launcher.cu:67-142
std::tuple<at::Tensor, at::Tensor, at::Tensor> flash_attention_bwd(at::Tensor Q, at::Tensor K,
                                                                   at::Tensor V, at::Tensor O,
                                                                   at::Tensor dO, at::Tensor L,
                                                                   bool causal) {
  TORCH_CHECK(Q.dim() == 4, "Q must be a 4D tensor (B, nh, T, hs)");
  const int64_t B = Q.size(0), nh = Q.size(1), T = Q.size(2), hs = Q.size(3);
  TORCH_CHECK(Q.is_cuda(), "Q must be a CUDA tensor");
  TORCH_CHECK(K.is_cuda(), "K must be a CUDA tensor");
  TORCH_CHECK(V.is_cuda(), "V must be a CUDA tensor");
  TORCH_CHECK(O.is_cuda(), "O must be a CUDA tensor");
  TORCH_CHECK(dO.is_cuda(), "dO must be a CUDA tensor");
  TORCH_CHECK(L.is_cuda(), "L must be a CUDA tensor");
  if (is_half16(Q)) return flash_attention_bwd_half(Q, K, V, O, dO, L, causal);
  for (const auto* t : {&Q, &K, &V, &O, &dO, &L}) check_f32(*t, "input");
  TORCH_CHECK(K.sizes() == Q.sizes() && V.sizes() == Q.sizes() && O.sizes() == Q.sizes() &&
                  dO.sizes() == Q.sizes(),
              "Q, K, V, O and dO must have the same shape");
  TORCH_CHECK(L.dim() == 3 && L.size(0) == B && L.size(1) == nh && L.size(2) == T,
              "L must be (B, nh, T)");
  c10::OptionalDeviceGuard guard(Q.device());
  at::Tensor dQ = at::empty({B, nh, T, hs}, Q.options());
  at::Tensor dK = at::empty({B, nh, T, hs}, Q.options());
  at::Tensor dV = at::empty({B, nh, T, hs}, Q.options());
  at::Tensor delta = at::empty({B, nh, T}, Q.options());
  if (hs != 32 && hs != 64 && hs != 128)
    TORCH_CHECK(false, "Unsupported head dimension! Only hs=32, hs=64, and hs=128 are supported.");
  const at::Tensor q = attn_operand(Q), k = attn_operand(K), v = attn_operand(V),
                   o = attn_operand(O), g = attn_operand(dO);
  const auto qs = strides_of<4>(q), ks = strides_of<4>(k), vs = strides_of<4>(v),
             os = strides_of<4>(o), gs = strides_of<4>(g);
  const auto ls = strides_of<3>(L);
  int64_t ws_bytes = 0;
  const at::Tensor ws = bwd_workspace(B, nh, T, hs, causal, Q.options(), ws_bytes);
  check_rc(cta_flash_attention_bwd(q.data_ptr<float>(), qs.data(), k.data_ptr<float>(), ks.data(),
                                   v.data_ptr<float>(), vs.data(), o.data_ptr<float>(), os.data(),
                                   g.data_ptr<float>(), gs.data(), L.data_ptr<float>(), ls.data(),
                                   B, nh, T, hs, causal ? 1 : 0, dQ.data_ptr<float>(),
                                   dK.data_ptr<float>(), dV.data_ptr<float>(),
                                   delta.data_ptr<float>(),
                                   ws_bytes > 0 ? ws.data_ptr<float>() : nullptr, ws_bytes,
                                   stream_of(Q)));
  return {dQ, dK, dV};
}

// ------------------------------------------------------------------ packed-qkv FlashAttention-2
// New ops with no reference counterpart: the attention of a packed (B, T, 3C) projection
// (C = nh * hs; Q, K, V its three column blocks, head h in columns h*hs .. h*hs + hs - 1 of
// each), as gpt.py:104-107 slices it, with the output O in the same head-interleaved (B, T, C)
// order and the gradient as one (B, T, 3C) tensor.  The kernels read the column blocks in place
// and write O and dQ/dK/dV through strides, so the head transposes, the copies behind them and
// the concatenation of dq, dk and dv disappear.  Same kernels and results as
// flash_attention_fwd / flash_attention_bwd on the head views.

// A packed (B, T, X) attention tensor read in place: unit last stride, strides divisible by 4,
// 16-byte aligned, time stride in [0, 2^23) (the kernels' 32-bit stage offsets).  Anything else
// is passed as a dense copy.
at::Tensor packed_operand(const at::Tensor& t) {
  const bool ok = t.stride(2) == 1 && t.stride(0) % 4 == 0 && t.stride(1) % 4 == 0 &&
                  t.stride(1) >= 0 && t.stride(1) < ((int64_t)1 << 23) &&
                  (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) == 0;
  return ok ? t : dense(t);
}

int64_t packed_head_size(const at::Tensor& qkv, int64_t nh) {
  TORCH_CHECK(qkv.dim() == 3, "qkv must be a 3D tensor (B, T, 3C)");
  TORCH_CHECK(qkv.is_cuda(), "qkv must be a CUDA tensor");
  check_f32(qkv, "qkv");
  TORCH_CHECK(nh > 0 && qkv.size(2) % (3 * nh) == 0, "qkv.size(2) must be 3 * nh * hs");
  const int64_t hs = qkv.size(2) / (3 * nh);
  if (hs != 32 && hs != 64 && hs != 128)
    TORCH_CHECK(false, "Unsupported head dimension! Only hs=32, hs=64, and hs=128 are supported.");
  return hs;
}

std::tuple<at::Tensor, at::Tensor> flash_attention_qkv_fwd(at::Tensor qkv, int64_t nh,
                                                           bool causal) {
  const int64_t hs = packed_head_size(qkv, nh);
  const int64_t B = qkv.size(0), T = qkv.size(1), C = nh * hs;
  c10::OptionalDeviceGuard guard(qkv.device());
  at::Tensor out = at::empty({B, T, C}, qkv.options());
  at::Tensor L = at::empty({B, nh, T}, qkv.options());
  const at::Tensor x = packed_operand(qkv);
  const float* p = x.data_ptr<float>();
  const int64_t xs[4] = {x.stride(0), hs, x.stride(1), 1};  // one column block as (B, nh, T, hs)
  const int64_t os[4] = {T * C, hs, C, 1};
  int64_t ws_bytes = 0;
  const at::Tensor ws = fwd_workspace(B, nh, T, hs, causal, qkv.options(), ws_bytes);
  check_rc(cta_flash_attention_fwd_ex(p, xs, p + C, xs, p + 2 * C, xs, B, nh, T, hs,
                                      causal ? 1 : 0, out.data_ptr<float>(), os,
                                      L.data_ptr<float>(), ws_bytes > 0 ? ws.data_ptr() : nullptr,
                                      ws_bytes, stream_of(qkv)));
  return {out, L};
}

at::Tensor flash_attention_qkv_bwd(at::Tensor qkv, at::Tensor out, at::Tensor dout,
                                   at::Tensor L, int64_t nh, bool causal) {
  const int64_t hs = packed_head_size(qkv, nh);
  const int64_t B = qkv.size(0), T = qkv.size(1), C = nh * hs;
  TORCH_CHECK(out.is_cuda() && dout.is_cuda() && L.is_cuda(),
              "out, dout and L must be CUDA tensors");
  for (const auto* t : {&out, &dout, &L}) check_f32(*t, "input");
  TORCH_CHECK(out.dim() == 3 && out.size(0) == B && out.size(1) == T && out.size(2) == C &&
                  dout.sizes() == out.sizes(),
              "out and dout must be (B, T, C)");
  TORCH_CHECK(L.dim() == 3 && L.size(0) == B && L.size(1) == nh && L.size(2) == T,
              "L must be (B, nh, T)");
  c10::OptionalDeviceGuard guard(qkv.device());
  at::Tensor dqkv = at::empty({B, T, 3 * C}, qkv.options());
  at::Tensor delta = at::empty({B, nh, T}, qkv.options());
  const at::Tensor x = packed_operand(qkv), o = packed_operand(out), g = packed_operand(dout);
  const float* p = x.data_ptr<float>();
  float* d = dqkv.data_ptr<float>();
  const int64_t xs[4] = {x.stride(0), hs, x.stride(1), 1};
  const int64_t os[4] = {o.stride(0), hs, o.stride(1), 1};
  const int64_t gs[4] = {g.stride(0), hs, g.stride(1), 1};
  const int64_t ds[4] = {T * 3 * C, hs, 3 * C, 1};
  const auto ls = strides_of<3>(L);
  int64_t ws_bytes = 0;
  const at::Tensor ws = bwd_workspace(B, nh, T, hs, causal, qkv.options(), ws_bytes);
  check_rc(cta_flash_attention_bwd_strided(
      p, xs, p + C, xs, p + 2 * C, xs, o.data_ptr<float>(), os, g.data_ptr<float>(), gs,
      L.data_ptr<float>(), ls.data(), B, nh, T, hs, causal ? 1 : 0, d, ds, d + C, ds, d + 2 * C,
      ds, delta.data_ptr<float>(), ws_bytes > 0 ? ws.data_ptr<float>() : nullptr, ws_bytes,
      stream_of(qkv)));
  return dqkv;
}

}  // namespace

TORCH_LIBRARY(cuda_transformer, m) {
  m.def("cuda_fma(Tensor x, Tensor weights, Tensor bias) -> Tensor");
  m.def("db_calculation(Tensor dy) -> Tensor");
  m.def("linear_weight_bias_grad(Tensor x, Tensor dy) -> (Tensor, Tensor)");
  m.def("cuda_fma_gelu(Tensor x, Tensor weights, Tensor bias) -> (Tensor, Tensor)");
  m.def("cuda_fma_gelu_grad(Tensor dy, Tensor weights, Tensor pre) -> Tensor");
  m.def("cuda_fma_gelu_tanh(Tensor x, Tensor weights, Tensor bias) -> (Tensor, Tensor)");
  m.def("cuda_fma_gelu_tanh_grad(Tensor dy, Tensor weights, Tensor pre) -> Tensor");
  m.def("cuda_fma_gelu_deriv(Tensor x, Tensor weights, Tensor bias) -> (Tensor, Tensor)");
  m.def("cuda_fma_gelu_tanh_deriv(Tensor x, Tensor weights, Tensor bias) -> (Tensor, Tensor)");
  m.def("cuda_fma_mul(Tensor dy, Tensor weights, Tensor d) -> Tensor");
  m.def("gelu_activation(Tensor x) -> Tensor");
  m.def("gelu_activation_bwd(Tensor x, Tensor dy) -> Tensor");
  m.def("gelu_tanh_activation(Tensor x) -> Tensor");
  m.def("gelu_tanh_activation_bwd(Tensor x, Tensor dy) -> Tensor");
  m.def("cuda_softmax(Tensor x) -> Tensor");
  m.def("cuda_softmax_bwd(Tensor probs, Tensor dp) -> Tensor");
  m.def("causal_self_attention_fwd(Tensor qkv, int nh, bool causal) -> (Tensor, Tensor)");
  m.def(
      "causal_self_attention_bwd(Tensor Q, Tensor K, Tensor V, Tensor probs, Tensor dO) -> "
      "(Tensor, Tensor, Tensor)");
  m.def("flash_attention_fwd(Tensor Q, Tensor K, Tensor V, bool causal) -> (Tensor, Tensor)");
  m.def(
      "flash_attention_bwd(Tensor Q, Tensor K, Tensor V, Tensor O, Tensor dO, Tensor L, bool "
      "causal) -> (Tensor, Tensor, Tensor)");
  m.def("flash_attention_qkv_fwd(Tensor qkv, int nh, bool causal) -> (Tensor, Tensor)");
  m.def(
      "flash_attention_qkv_bwd(Tensor qkv, Tensor out, Tensor dout, Tensor L, int nh, bool "
      "causal) -> Tensor");
  m.def("layernorm_fwd(Tensor x, Tensor gamma, Tensor beta, float eps) -> (Tensor, Tensor, Tensor)");
  m.def("add_layernorm_fwd(Tensor x, Tensor f, Tensor gamma, Tensor beta, float eps) -> "
        "(Tensor, Tensor, Tensor, Tensor)");
  m.def("add_layernorm_bwd(Tensor xsum, Tensor gamma, Tensor mean, Tensor rstd, Tensor dy, "
        "Tensor dres) -> (Tensor, Tensor, Tensor)");
  m.def(
      "layernorm_bwd(Tensor x, Tensor gamma, Tensor mean, Tensor rstd, Tensor dy) -> "
      "(Tensor, Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(cuda_transformer, CUDA, m) {
  m.impl("cuda_fma", &cuda_fma);
  m.impl("db_calculation", &db_calculation);
  m.impl("linear_weight_bias_grad", &linear_weight_bias_grad);
  m.impl("cuda_fma_gelu", &cuda_fma_gelu);
  m.impl("cuda_fma_gelu_grad", &cuda_fma_gelu_grad);
  m.impl("cuda_fma_gelu_tanh", &cuda_fma_gelu_tanh);
  m.impl("cuda_fma_gelu_tanh_grad", &cuda_fma_gelu_tanh_grad);
  m.impl("cuda_fma_gelu_deriv", &cuda_fma_gelu_deriv);
  m.impl("cuda_fma_gelu_tanh_deriv", &cuda_fma_gelu_tanh_deriv);
  m.impl("cuda_fma_mul", &cuda_fma_mul);
  m.impl("gelu_activation", &gelu_activation);
  m.impl("gelu_activation_bwd", &gelu_activation_bwd);
  m.impl("gelu_tanh_activation", &gelu_tanh_activation);
  m.impl("gelu_tanh_activation_bwd", &gelu_tanh_activation_bwd);
  m.impl("cuda_softmax", &cuda_softmax);
  m.impl("cuda_softmax_bwd", &cuda_softmax_bwd);
  m.impl("causal_self_attention_fwd", &causal_self_attention_fwd);
  m.impl("causal_self_attention_bwd", &causal_self_attention_bwd);
  m.impl("flash_attention_fwd", &flash_attention_fwd);
  m.impl("flash_attention_bwd", &flash_attention_bwd);
  m.impl("flash_attention_qkv_fwd", &flash_attention_qkv_fwd);
  m.impl("flash_attention_qkv_bwd", &flash_attention_qkv_bwd);
  m.impl("layernorm_fwd", &layernorm_fwd);
  m.impl("layernorm_bwd", &layernorm_bwd);
  m.impl("add_layernorm_fwd", &add_layernorm_fwd);
  m.impl("add_layernorm_bwd", &add_layernorm_bwd);
}

}  // namespace cuda_transformer

// Importable as cuda_transformer_amd._C (the reference imports cuda_transformer._C); importing
// it runs the static registrations above.
namespace {
PyObject* py_last_bwd_schedule(PyObject*, PyObject*) {
  const int s = cuda_transformer::last_bwd_schedule().load();
  return PyUnicode_FromString(s == 1 ? "stored" : s == 0 ? "recompute" : "none");
}
PyObject* py_bwd_workspace_cap(PyObject*, PyObject*) {
  return PyLong_FromLongLong(cuda_transformer::bwd_workspace_cap().load());
}
PyObject* py_set_bwd_workspace_cap(PyObject*, PyObject* arg) {
  const long long v = PyLong_AsLongLong(arg);
  if (v == -1 && PyErr_Occurred()) return nullptr;
  if (v < 0) {
    PyErr_SetString(PyExc_ValueError, "the workspace cap must be a byte count >= 0");
    return nullptr;
  }
  return PyLong_FromLongLong(cuda_transformer::bwd_workspace_cap().exchange(v));
}
PyMethodDef kMethods[] = {
    {"last_bwd_schedule", py_last_bwd_schedule, METH_NOARGS,
     "Backward schedule of the last flash_attention_bwd in this process: 'stored' (dK/dV "
     "stores dS, dQ reads it), 'recompute' (no dS workspace: the 16-bit default at hs 32 and "
     "64, a cap below one head, or not allocatable) or 'none'."},
    {"bwd_workspace_cap", py_bwd_workspace_cap, METH_NOARGS,
     "Largest dS workspace, in bytes, that flash_attention_bwd allocates (default 8 GiB)."},
    {"set_bwd_workspace_cap", py_set_bwd_workspace_cap, METH_O,
     "Set the dS workspace cap in bytes and return the previous one.  Heads whose dS tiles do "
     "not all fit run in chunks; below one head (e.g. 0) the backward recomputes S and dP in "
     "its dQ stage and allocates no workspace.  Process-wide."},
    {nullptr, nullptr, 0, nullptr}};
}  // namespace

extern "C" PyObject* PyInit__C(void) {
  static struct PyModuleDef def = {PyModuleDef_HEAD_INIT, "_C",
                                   "gfx950 FP32 transformer kernels: torch operator library",
                                   -1, kMethods, nullptr, nullptr, nullptr, nullptr};
  return PyModule_Create(&def);
}
