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

// Pointwise stage applied to v = alpha * acc + bias before the store.
enum GemmAct {
  kActNone = 0,
  kActGelu = 1,      // C = v (the pre-activation) and aux = gelu(v)
  kActGeluGrad = 2,  // C = v * gelu'(aux): aux holds the pre-activation
  kActGeluTanh = 3,      // as kActGelu with the tanh-approximated GELU
  kActGeluTanhGrad = 4,  // as kActGeluGrad with the tanh-approximated GELU
  kActGeluDeriv = 5,      // C = gelu'(v) and aux = gelu(v)
  kActGeluTanhDeriv = 6,  // as kActGeluDeriv with the tanh-approximated GELU
  kActMulAux = 7,         // C = v * aux: aux holds a saved gelu'(pre)
};

struct GemmEpilogue {
  float alpha;
  const float* bias;  // nullable, indexed by n
  int64_t bias_stride;
  int causal_mask;    // set entries with n > m to -inf
  int act = kActNone;
  float* aux = nullptr;  // same (batch, m, n) layout as the output; read-only for the *Grad acts and kActMulAux
  // Nullable: receives the column sums of B over K (sum_k B[k][n], n < N).  Needs Z == 1,
  // B contiguous along n with N % 4 == 0, no pointwise stage and no mask.
  float* colsum = nullptr;
};

// out[z] = alpha * A[z] B[z] (+ bias) for z in [0, Z); batch index split as (z / zin, z % zin).
// With a workspace of gemm_workspace_floats(M, N, K, Z) floats, shapes with too few output
// tiles to fill the GPU are split along K (deterministic fixed-order reduction).
// With ep.colsum the split-K workspace also holds one row of column sums per split:
// gemm_workspace_floats(M, N, K, Z, true) floats.
int gemm_launch(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z, int64_t zin,
                hipStream_t st, float* workspace = nullptr, int64_t workspace_floats = 0);
int64_t gemm_workspace_floats(int64_t M, int64_t N, int64_t K, int64_t Z, bool colsum = false);

// Row softmax over `rows` dense rows of length n (x == y allowed).
int softmax_rows(const float* x, float* y, int64_t rows, int64_t n, hipStream_t st);
// dx = p * (dp - rowsum(p * dp)) over dense rows (dx may alias dp or p).
int softmax_bwd_rows_launch(const float* p, const float* dp, float* dx, int64_t rows, int64_t n,
                            hipStream_t st);

// Column sums of a strided (batch, M, N) tensor into out[N]; workspace holds
// colsum_workspace_floats(batch * M, N) floats.  Deterministic.
int colsum_launch(const float* x, int64_t batch, int64_t M, int64_t N, int64_t sb, int64_t sm,
                  int64_t sn, float* out, float* workspace, hipStream_t st);
int64_t colsum_chunks(int64_t rows);
int64_t colsum_workspace_floats(int64_t rows, int64_t N);
// Fixed-order sum over the rows of part[chunks][ncols]: column c goes to out0[c] (c < split)
// or out1[c - split].  `scratch` (colsum_partials_scratch_floats floats, may be null) lets the
// sum run in two parallel stages.
int colsum_partials_launch(const float* part, int64_t chunks, int64_t ncols, float* out0,
                           float* out1, int64_t split, hipStream_t st, float* scratch);
int64_t colsum_partials_scratch_floats(int64_t chunks, int64_t ncols);

}  // namespace cta
