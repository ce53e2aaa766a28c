// Internal interface of the strided batched GEMM and the row softmax, shared by the
// linear-layer entry points and the naive attention.
#pragma once

#include "cta_common.hpp"

namespace cta {

struct GemmOperand {
  const float* p;
  int64_t s_outer, s_inner;  // batch strides (z / zin, z % zin)
  int64_t s_row, s_col;      // A: (m, k)   B: (k, n)
};

struct GemmOut {
  float* p;
  int64_t s_outer, s_inner, s_row;  // column stride is 1
};

struct GemmEpilogue {
  float alpha;
  const float* bias;  // nullable, indexed by n
  int64_t bias_stride;
  int causal_mask;    // set entries with n > m to -inf
};

// out[z] = alpha * A[z] B[z] (+ bias) for z in [0, Z); batch index split as (z / zin, z % zin).
int gemm_launch(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z, int64_t zin,
                hipStream_t st);

// Row softmax over `rows` dense rows of length n (x == y allowed).
int softmax_rows(const float* x, float* y, int64_t rows, int64_t n, hipStream_t st);
// dx = p * (dp - rowsum(p * dp)) over dense rows (dx may alias dp or p).
int softmax_bwd_rows_launch(const float* p, const float* dp, float* dx, int64_t rows, int64_t n,
                            hipStream_t st);

}  // namespace cta
