// Materialised ("naive") causal self-attention, FP32, built from the strided batched MFMA
// GEMM and the register-resident row softmax.
//
// Forward follows Transformer_launchers/causal_self_attn_layer.cu:24-67:
//   S = (Q K^T) / sqrt(hs) with -inf above the diagonal when causal, read straight out of the
//   packed qkv (B, T, 3C) tensor (causal_self_attention_fwd.cuh:9-67); softmax over S in place
//   (softmax.cuh:25-106); out = P V written into (B, T, C) (causal_self_attention_fwd.cuh:69-127).
//   Returns (out, probs) with probs (B, nh, T, T).
// Backward follows causal_self_attn_layer.cu:70-132 on (B*nh, T, hs) operands:
//   dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(P dP)), dQ = dS K, dK = dS^T Q.
//   dQ and dK are returned unscaled; the caller divides them by sqrt(hs).
#include "cta_common.hpp"
#include "gemm.hpp"

using namespace cta;

extern "C" int cta_causal_self_attention_fwd(const float* qkv, int64_t B, int64_t T, int64_t C,
                                             int64_t nh, int causal, float* out, float* probs,
                                             void* stream) {
  if (B < 0 || T < 0 || C < 0 || nh <= 0) return fail(CTA_ERR_INVALID_ARGUMENT, "bad size");
  if (C % nh != 0) return fail(CTA_ERR_INVALID_ARGUMENT, "C must be divisible by nh");
  if (B * T * C == 0) return CTA_OK;
  if (!qkv || !out || !probs) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  const int64_t hs = C / nh;
  hipStream_t st = as_stream(stream);
  // S[b,h] = Q[b,h] K[b,h]^T * (1/sqrt(hs)): batch z = b*nh + h.
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const GemmOperand Aq{qkv, T * 3 * C, hs, 3 * C, 1};
  const GemmOperand Bk{qkv + C, T * 3 * C, hs, 1, 3 * C};  // (k=d, n=j) -> K[j][d]
  const GemmOut S{probs, nh * T * T, T * T, T};
  const GemmEpilogue ep_s{scale, nullptr, 0, causal ? 1 : 0};
  if (int rc = gemm_launch(Aq, Bk, S, ep_s, T, T, hs, B * nh, nh, st)) return rc;
  if (int rc = softmax_rows(probs, probs, B * nh * T, T, st)) return rc;
  // out[b, t, h*hs + d] = sum_j P[b,h,t,j] V[b,j,h*hs+d]
  const GemmOperand Ap{probs, nh * T * T, T * T, T, 1};
  const GemmOperand Bv{qkv + 2 * C, T * 3 * C, hs, 3 * C, 1};
  const GemmOut O{out, T * C, hs, C};
  const GemmEpilogue ep_o{1.0f, nullptr, 0, 0};
  return gemm_launch(Ap, Bv, O, ep_o, T, hs, T, B * nh, nh, st);
}

extern "C" int64_t cta_causal_self_attention_bwd_workspace(int64_t BH, int64_t T) {
  if (BH <= 0 || T <= 0) return 0;
  return BH * T * T * (int64_t)sizeof(float);
}

extern "C" int cta_causal_self_attention_bwd(const float* q, const int64_t* q_strides,
                                             const float* k, const int64_t* k_strides,
                                             const float* v, const int64_t* v_strides,
                                             const float* probs, const float* d_o,
                                             const int64_t* do_strides, int64_t BH, int64_t T,
                                             int64_t hs, float* dq, float* dk, float* dv,
                                             float* workspace, void* stream) {
  if (BH < 0 || T < 0 || hs < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (BH * T * hs == 0) return CTA_OK;
  if (!q || !k || !v || !probs || !d_o || !dq || !dk || !dv || !workspace || !q_strides ||
      !k_strides || !v_strides || !do_strides)
    return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  hipStream_t st = as_stream(stream);
  const GemmEpilogue plain{1.0f, nullptr, 0, 0};
  const int64_t TT = T * T;
  // dV = P^T dO : A[m=j][k=i] = P[i][j]
  const GemmOperand Apt{probs, TT, 0, 1, T};
  const GemmOperand Bdo{d_o, do_strides[0], 0, do_strides[1], do_strides[2]};
  const GemmOut Odv{dv, T * hs, 0, hs};
  if (int rc = gemm_launch(Apt, Bdo, Odv, plain, T, hs, T, BH, 1, st)) return rc;
  // dP = dO V^T : B[k=d][n=j] = V[j][d]
  const GemmOperand Ado{d_o, do_strides[0], 0, do_strides[1], do_strides[2]};
  const GemmOperand Bvt{v, v_strides[0], 0, v_strides[2], v_strides[1]};
  const GemmOut Odp{workspace, TT, 0, T};
  if (int rc = gemm_launch(Ado, Bvt, Odp, plain, T, T, hs, BH, 1, st)) return rc;
  // dS = P (dP - rowsum(P dP)), in place over dP
  if (int rc = softmax_bwd_rows_launch(probs, workspace, workspace, BH * T, T, st)) return rc;
  // dQ = dS K
  const GemmOperand Ads{workspace, TT, 0, T, 1};
  const GemmOperand Bk{k, k_strides[0], 0, k_strides[1], k_strides[2]};
  const GemmOut Odq{dq, T * hs, 0, hs};
  if (int rc = gemm_launch(Ads, Bk, Odq, plain, T, hs, T, BH, 1, st)) return rc;
  // dK = dS^T Q : A[m=j][k=i] = dS[i][j]
  const GemmOperand Adst{workspace, TT, 0, 1, T};
  const GemmOperand Bq{q, q_strides[0], 0, q_strides[1], q_strides[2]};
  const GemmOut Odk{dk, T * hs, 0, hs};
  return gemm_launch(Adst, Bq, Odk, plain, T, hs, T, BH, 1, st);
}
