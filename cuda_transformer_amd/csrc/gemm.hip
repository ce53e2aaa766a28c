// The strided, batched FP32 GEMM's tile choice and the linear layer's C entry points (kernels:
// gemm_kernel.hpp; instances: gemm_tiles_*.hip).
#include "gemm_kernel.hpp"

namespace cta {

int64_t gemm_workspace_floats(int64_t M, int64_t N, int64_t K, int64_t Z, bool colsum) {
  const int64_t S = splitk_factor<SplitTile>(M, N, K, Z);
  return S > 1 ? S * (Z * M * N + (colsum ? N : 0)) : 0;
}

// Launch the strided batched GEMM.  Z = number of batches, zin = inner batch extent.  With a
// workspace of gemm_workspace_floats() floats, low-parallelism shapes are split along K.
int gemm_launch(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z, int64_t zin,
                hipStream_t st, float* workspace, int64_t workspace_floats) {
  const int64_t S = splitk_factor<SplitTile>(M, N, K, Z);
  if (S > 1 && workspace != nullptr &&
      workspace_floats >= S * (Z * M * N + (ep.colsum ? N : 0)))
    return gemm_launch_split(A, B, C, ep, M, N, K, Z, zin, st, workspace, workspace_floats);
  // A product's tile never depends on its pointwise stage alone, except between the two wide
  // tiles, which share their K-slice (hence the k pairs each MFMA sums): a fused GELU product
  // stays bitwise equal to the plain product followed by the GELU kernel.
  const bool n192 = N % 192 == 0;
  if (N <= 768) {
    if (n192 && K <= 512)
      return gemm_launch_narrow192_short_k(A, B, C, ep, M, N, K, Z, zin, st, nullptr, 0);
    if (n192) return gemm_launch_narrow192(A, B, C, ep, M, N, K, Z, zin, st, nullptr, 0);
    return gemm_launch_narrow(A, B, C, ep, M, N, K, Z, zin, st, nullptr, 0);
  }
  if (n192 && ep.act == kActNone)
    return gemm_launch_wide192(A, B, C, ep, M, N, K, Z, zin, st, nullptr, 0);
  return gemm_launch_wide(A, B, C, ep, M, N, K, Z, zin, st, nullptr, 0);
}

}  // namespace cta

using namespace cta;

extern "C" int64_t cta_cuda_fma_workspace(int64_t batch, int64_t m, int64_t k, int64_t n) {
  if (batch <= 0 || m <= 0 || n <= 0 || k <= 0) return 0;
  return gemm_workspace_floats(m, n, k, batch) * (int64_t)sizeof(float);
}

namespace {
// out[b] = x[b] . W[b or 0] with epilogue `ep`, out dense (batch, m, n): the shared body of the
// linear-layer entry points.  Weights broadcast over the batch with batch stride 0 when
// w_batch == 1, as linear_layer.cu:30-34 does.
int linear_launch(const float* x, const int64_t* x_strides, const float* w,
                  const int64_t* w_strides, int64_t batch, int64_t m, int64_t k, int64_t n,
                  int64_t w_batch, float* out, const GemmEpilogue& ep, float* workspace,
                  void* stream) {
  if (batch < 0 || m < 0 || k < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (w_batch != 1 && w_batch != batch)
    return fail(CTA_ERR_INVALID_ARGUMENT, "weights batch must be 1 or equal to x batch");
  if (batch * m * n == 0) return CTA_OK;
  if (!x || !w || !out || !x_strides || !w_strides)
    return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  const GemmOperand A{x, x_strides[0], 0, x_strides[1], x_strides[2]};
  const GemmOperand B{w, w_batch == 1 ? 0 : w_strides[0], 0, w_strides[1], w_strides[2]};
  const GemmOut C{out, m * n, 0, n};
  return gemm_launch(A, B, C, ep, m, n, k, batch, 1, as_stream(stream), workspace,
                     workspace ? gemm_workspace_floats(m, n, k, batch) : 0);
}
}  // namespace

extern "C" int cta_cuda_fma(const float* x, const int64_t* x_strides, const float* w,
                            const int64_t* w_strides, const float* bias, int64_t bias_stride,
                            int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                            float* out, float* workspace, void* stream) {
  if (!bias && batch > 0 && m > 0 && n > 0) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  const GemmEpilogue ep{1.0f, bias, bias_stride, 0};
  return linear_launch(x, x_strides, w, w_strides, batch, m, k, n, w_batch, out, ep, workspace,
                       stream);
}

namespace {
int fma_act(const float* x, const int64_t* x_strides, const float* w, const int64_t* w_strides,
            const float* bias, int64_t bias_stride, int64_t batch, int64_t m, int64_t k,
            int64_t n, int64_t w_batch, float* pre, float* out, float* workspace, void* stream,
            int act) {
  if (batch > 0 && m > 0 && n > 0) {
    if (!bias || !out) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
    if (pre == out) return fail(CTA_ERR_INVALID_ARGUMENT, "pre and out must be distinct buffers");
  }
  const GemmEpilogue ep{1.0f, bias, bias_stride, 0, act, out};
  return linear_launch(x, x_strides, w, w_strides, batch, m, k, n, w_batch, pre, ep, workspace,
                       stream);
}

int fma_act_grad(const float* dy, const int64_t* dy_strides, const float* w,
                 const int64_t* w_strides, const float* pre, int64_t batch, int64_t m, int64_t k,
                 int64_t n, int64_t w_batch, float* dx, float* workspace, void* stream, int act) {
  if (!pre && batch > 0 && m > 0 && n > 0) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  // Each output element reads its own pre-activation just before it is stored, so dx may
  // alias pre.
  const GemmEpilogue ep{1.0f, nullptr, 0, 0, act, const_cast<float*>(pre)};
  return linear_launch(dy, dy_strides, w, w_strides, batch, m, k, n, w_batch, dx, ep, workspace,
                       stream);
}
}  // namespace

extern "C" int cta_cuda_fma_gelu(const float* x, const int64_t* x_strides, const float* w,
                                 const int64_t* w_strides, const float* bias,
                                 int64_t bias_stride, int64_t batch, int64_t m, int64_t k,
                                 int64_t n, int64_t w_batch, float* pre, float* out,
                                 float* workspace, void* stream) {
  return fma_act(x, x_strides, w, w_strides, bias, bias_stride, batch, m, k, n, w_batch, pre, out,
                 workspace, stream, kActGelu);
}

extern "C" int cta_cuda_fma_gelu_grad(const float* dy, const int64_t* dy_strides, const float* w,
                                      const int64_t* w_strides, const float* pre, int64_t batch,
                                      int64_t m, int64_t k, int64_t n, int64_t w_batch,
                                      float* dx, float* workspace, void* stream) {
  return fma_act_grad(dy, dy_strides, w, w_strides, pre, batch, m, k, n, w_batch, dx, workspace,
                      stream, kActGeluGrad);
}

extern "C" int cta_cuda_fma_gelu_tanh(const float* x, const int64_t* x_strides, const float* w,
                                      const int64_t* w_strides, const float* bias,
                                      int64_t bias_stride, int64_t batch, int64_t m, int64_t k,
                                      int64_t n, int64_t w_batch, float* pre, float* out,
                                      float* workspace, void* stream) {
  return fma_act(x, x_strides, w, w_strides, bias, bias_stride, batch, m, k, n, w_batch, pre, out,
                 workspace, stream, kActGeluTanh);
}

extern "C" int cta_cuda_fma_gelu_tanh_grad(const float* dy, const int64_t* dy_strides,
                                           const float* w, const int64_t* w_strides,
                                           const float* pre, int64_t batch, int64_t m, int64_t k,
                                           int64_t n, int64_t w_batch, float* dx,
                                           float* workspace, void* stream) {
  return fma_act_grad(dy, dy_strides, w, w_strides, pre, batch, m, k, n, w_batch, dx, workspace,
                      stream, kActGeluTanhGrad);
}

extern "C" int cta_cuda_fma_gelu_deriv(const float* x, const int64_t* x_strides, const float* w,
                                       const int64_t* w_strides, const float* bias,
                                       int64_t bias_stride, int64_t batch, int64_t m, int64_t k,
                                       int64_t n, int64_t w_batch, float* deriv, float* out,
                                       float* workspace, void* stream) {
  return fma_act(x, x_strides, w, w_strides, bias, bias_stride, batch, m, k, n, w_batch, deriv,
                 out, workspace, stream, kActGeluDeriv);
}

extern "C" int cta_cuda_fma_gelu_tanh_deriv(const float* x, const int64_t* x_strides,
                                            const float* w, const int64_t* w_strides,
                                            const float* bias, int64_t bias_stride,
                                            int64_t batch, int64_t m, int64_t k, int64_t n,
                                            int64_t w_batch, float* deriv, float* out,
                                            float* workspace, void* stream) {
  return fma_act(x, x_strides, w, w_strides, bias, bias_stride, batch, m, k, n, w_batch, deriv,
                 out, workspace, stream, kActGeluTanhDeriv);
}

extern "C" int cta_cuda_fma_mul(const float* dy, const int64_t* dy_strides, const float* w,
                                const int64_t* w_strides, const float* d, int64_t batch,
                                int64_t m, int64_t k, int64_t n, int64_t w_batch, float* dx,
                                float* workspace, void* stream) {
  return fma_act_grad(dy, dy_strides, w, w_strides, d, batch, m, k, n, w_batch, dx, workspace,
                      stream, kActMulAux);
}

extern "C" int64_t cta_db_calculation_workspace(int64_t batch, int64_t m, int64_t n) {
  if (batch <= 0 || m <= 0 || n <= 0) return 0;
  return colsum_workspace_floats(batch * m, n) * (int64_t)sizeof(float);
}

extern "C" int cta_db_calculation(const float* dy, const int64_t* dy_strides, int64_t batch,
                                  int64_t m, int64_t n, float* db, float* workspace,
                                  void* stream) {
  if (batch < 0 || m < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (n == 0) return CTA_OK;
  if (!db) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  hipStream_t st = as_stream(stream);
  if (batch * m == 0) return zero_floats(db, n, st);
  if (!dy || !dy_strides || !workspace) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  return colsum_launch(dy, batch, m, n, dy_strides[0], dy_strides[1], dy_strides[2], db,
                       workspace, st);
}

extern "C" int64_t cta_linear_weight_bias_grad_workspace(int64_t rows, int64_t k, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  // k == 0: no GEMM, but db still comes from the column-sum kernels' partials
  if (k <= 0) return colsum_workspace_floats(rows, n) * (int64_t)sizeof(float);
  const int64_t fused = gemm_workspace_floats(k, n, rows, 1, true);
  const int64_t apart = std::max(gemm_workspace_floats(k, n, rows, 1), colsum_workspace_floats(rows, n));
  return std::max(fused, apart) * (int64_t)sizeof(float);
}

// dW = x^T dy as one GEMM over the rows (A = x^T through x's strides), with db = the column sums
// of dy taken from the GEMM's own dy slices when dy is n-contiguous with n % 4 == 0; otherwise
// the GEMM and then the column-sum kernels.
extern "C" int cta_linear_weight_bias_grad(const float* x, const int64_t* x_strides,
                                           const float* dy, const int64_t* dy_strides,
                                           int64_t rows, int64_t k, int64_t n, float* dw,
                                           float* db, float* workspace, void* stream) {
  if (rows < 0 || k < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (n == 0) return CTA_OK;
  if (!db || (k > 0 && !dw)) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    if (int rc = zero_floats(db, n, st)) return rc;
    return k > 0 ? zero_floats(dw, k * n, st) : CTA_OK;
  }
  if (!dy || !dy_strides || (k > 0 && (!x || !x_strides)))
    return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  const int64_t ws_floats = cta_linear_weight_bias_grad_workspace(rows, k, n) / (int64_t)sizeof(float);
  if (ws_floats > 0 && !workspace) return fail(CTA_ERR_INVALID_ARGUMENT, "null workspace");
  const GemmOperand B{dy, 0, 0, dy_strides[0], dy_strides[1]};
  const GemmOut C{dw, k * n, 0, n};
  GemmEpilogue ep{1.0f, nullptr, 0, 0};
  if (k > 0) {
    const GemmOperand A{x, 0, 0, x_strides[1], x_strides[0]};
    if (pick_mode(B, false, n, rows) == kVecMN) {
      ep.colsum = db;
      return gemm_launch(A, B, C, ep, k, n, rows, 1, 1, st, workspace, ws_floats);
    }
    if (int rc = gemm_launch(A, B, C, ep, k, n, rows, 1, 1, st, workspace, ws_floats)) return rc;
  }
  return colsum_launch(dy, 1, rows, n, 0, dy_strides[0], dy_strides[1], db, workspace, st);
}
