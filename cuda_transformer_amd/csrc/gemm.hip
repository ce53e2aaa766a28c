// Strided, batched FP32 GEMM on CDNA4 MFMA, and the linear layer's C entry points.
//
//   out[z][m][n] = alpha * sum_k A[z][m][k] * B[z][k][n]  (+ bias[n])  (causal: -inf for n > m)
//
// This one kernel backs the reference's fused_multiply_add (Transformer_kernels/
// fused_multiply_add.cuh:10-92, launched from Transformer_launchers/linear_layer.cu:28-70),
// its strided batched cuda_bmm (batched_matrix_multiply.cuh:9-75) and the two GEMM stages of
// the naive attention (causal_self_attention_fwd.cuh:9-127).  Every operand is addressed
// through strides, so transposed views (W^T, x^T in the linear backward) need no copies.
// The batch index z is split as (z / zin, z % zin) with a stride per level, which lets
// the naive attention address heads inside a packed (B, T, 3C) tensor directly.
//
// gfx950 design: 256 threads = 4 waves in a 2x2 arrangement; workgroup tile 128x128, wave
// tile 64x64 = 2x2 v_mfma_f32_32x32x2_f32 blocks.  A and B tiles are staged through LDS as
// [m][k] and [n][k] (k contiguous, pitch BK+4), so each MFMA operand fragment is a pair of
// conflict-free 16-byte LDS reads whatever the operand's memory order.  Global loads are
// dwordx4 along whichever dimension is contiguous in memory (template mode), with scalar
// loads for ragged edges and irregular strides.
#include "cta_common.hpp"
#include "gemm.hpp"

namespace cta {

enum LoadMode { kVecK = 0, kVecMN = 1, kScalar = 2 };

namespace {

constexpr int GBM = 128, GBN = 128, GBK = 16;
constexpr int GKP = GBK + 4;  // LDS pitch (floats) of one m (or n) row of a k-slice

// Loads one 128 x 16 slice of an operand into registers.  `rows` indexes m (A) or n (B);
// the operand is row-major in (row, k) when kVecK, (k, row) when kVecMN.
template <int MODE>
struct TileLoader {
  float4 v[2];
  __device__ __forceinline__ void load(const float* base, int64_t s_row, int64_t s_k, int row0,
                                       int k0, int R, int K, int tid) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int f = tid + 256 * u;
      if (MODE == kVecK) {
        const int r = f >> 2, k4 = (f & 3) * 4;
        const int gr = row0 + r, gk = k0 + k4;
        const float* p = base + (int64_t)gr * s_row + gk;
        if (gr < R && gk + 3 < K) {
          v[u] = ld4(p);
        } else {
          float t[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) t[e] = (gr < R && gk + e < K) ? p[e] : 0.0f;
          v[u] = make_float4(t[0], t[1], t[2], t[3]);
        }
      } else if (MODE == kVecMN) {
        const int k = f >> 5, r4 = (f & 31) * 4;
        const int gr = row0 + r4, gk = k0 + k;
        const float* p = base + (int64_t)gk * s_k + gr;
        if (gk < K && gr + 3 < R) {
          v[u] = ld4(p);
        } else {
          float t[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) t[e] = (gk < K && gr + e < R) ? p[e] : 0.0f;
          v[u] = make_float4(t[0], t[1], t[2], t[3]);
        }
      } else {
        const int r = f >> 2, k4 = (f & 3) * 4;
        const int gr = row0 + r;
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int gk = k0 + k4 + e;
          t[e] = (gr < R && gk < K) ? base[(int64_t)gr * s_row + (int64_t)gk * s_k] : 0.0f;
        }
        v[u] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
  }
  // LDS image: [row][k], pitch GKP.
  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int f = tid + 256 * u;
      if (MODE == kVecMN) {
        const int k = f >> 5, r4 = (f & 31) * 4;
        lds[(r4 + 0) * GKP + k] = v[u].x;
        lds[(r4 + 1) * GKP + k] = v[u].y;
        lds[(r4 + 2) * GKP + k] = v[u].z;
        lds[(r4 + 3) * GKP + k] = v[u].w;
      } else {
        const int r = f >> 2, k4 = (f & 3) * 4;
        st4(lds + r * GKP + k4, v[u]);
      }
    }
  }
};

// split_ws == nullptr: out = alpha * A B (+ bias, mask) written through C.
// split_ws != nullptr: blockIdx.z = s * Z + z covers K range [s*kchunk, (s+1)*kchunk) and the raw
// partial sum goes to split_ws[s][z][m][n] (dense); gemm_splitk_reduce finishes the epilogue.
template <int AMODE, int BMODE>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmOperand A, GemmOperand B, GemmOut C,
                                                      GemmEpilogue ep, int M, int N, int K,
                                                      int zin, int Z, int kchunk,
                                                      float* __restrict__ split_ws) {
  __shared__ __attribute__((aligned(16))) float smem[2 * (GBM + GBN) * GKP];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, col = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;

  const int n0 = blockIdx.x * GBN, m0 = blockIdx.y * GBM;
  const int z = blockIdx.z % Z, split = blockIdx.z / Z;
  const int zo = z / zin, zi = z - zo * zin;
  const float* Ab = A.p + zo * A.s_outer + zi * A.s_inner;
  const float* Bb = B.p + zo * B.s_outer + zi * B.s_inner;
  const int kb = split * kchunk;
  const int ke = min(K, kb + kchunk);

  // A rows are m with (s_row, s_col) = (m, k); B "rows" are n with (n, k) = (s_col, s_row).
  TileLoader<AMODE> la;
  TileLoader<BMODE> lb;
  const int nk = (ke - kb + GBK - 1) / GBK;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

  la.load(Ab, A.s_row, A.s_col, m0, kb, M, ke, tid);
  lb.load(Bb, B.s_col, B.s_row, n0, kb, N, ke, tid);
  la.store(smem, tid);
  lb.store(smem + GBM * GKP, tid);
  __syncthreads();

  for (int t = 0; t < nk; ++t) {
    const int buf = t & 1;
    if (t + 1 < nk) {
      la.load(Ab, A.s_row, A.s_col, m0, kb + (t + 1) * GBK, M, ke, tid);
      lb.load(Bb, B.s_col, B.s_row, n0, kb + (t + 1) * GBK, N, ke, tid);
    }
    const float* as = smem + buf * (GBM + GBN) * GKP;
    const float* bs = as + GBM * GKP;
    float4 af[2][2], bf[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float* ap = as + (wm * 64 + i * 32 + col) * GKP + half * (GBK / 2);
      const float* bp = bs + (wn * 64 + i * 32 + col) * GKP + half * (GBK / 2);
      af[i][0] = ld4(ap);
      af[i][1] = ld4(ap + 4);
      bf[i][0] = ld4(bp);
      bf[i][1] = ld4(bp + 4);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = mfma32(af[i][c].x, bf[j][c].x, acc[i][j]);
          acc[i][j] = mfma32(af[i][c].y, bf[j][c].y, acc[i][j]);
          acc[i][j] = mfma32(af[i][c].z, bf[j][c].z, acc[i][j]);
          acc[i][j] = mfma32(af[i][c].w, bf[j][c].w, acc[i][j]);
        }
    }
    if (t + 1 < nk) {
      float* nas = smem + (buf ^ 1) * (GBM + GBN) * GKP;
      la.store(nas, tid);
      lb.store(nas + GBM * GKP, tid);
    }
    __syncthreads();
  }

  if (split_ws != nullptr) {
    float* Pb = split_ws + ((int64_t)split * Z + z) * M * N;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 64 + j * 32 + col;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * 64 + i * 32 + mfma_row(r, half);
          if (m < M) Pb[(int64_t)m * N + n] = acc[i][j][r];
        }
    }
    return;
  }
  float* Cb = C.p + zo * C.s_outer + zi * C.s_inner;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn * 64 + j * 32 + col;
    if (n >= N) continue;
    const float bv = ep.bias ? ep.bias[(int64_t)n * ep.bias_stride] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * 64 + i * 32 + mfma_row(r, half);
        if (m < M) {
          float val = fmaf(ep.alpha, acc[i][j][r], bv);
          if (ep.causal_mask && n > m) val = -INFINITY;
          Cb[(int64_t)m * C.s_row + n] = val;
        }
      }
    }
  }
}

// Fixed-order sum of the split-K partials plus the epilogue of gemm_kernel.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float* __restrict__ ws, int S,
                                                          int Z, int M, int N, GemmOut C,
                                                          GemmEpilogue ep, int zin) {
  const int64_t total = (int64_t)Z * M * N;
  const int64_t plane = total;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * 256) {
    float acc = ws[e];
    for (int s = 1; s < S; ++s) acc += ws[(int64_t)s * plane + e];
    const int64_t z = e / ((int64_t)M * N);
    const int64_t mn = e - z * M * N;
    const int m = (int)(mn / N), n = (int)(mn - (int64_t)m * N);
    const int64_t zo = z / zin, zi = z - zo * zin;
    float val = fmaf(ep.alpha, acc, ep.bias ? ep.bias[(int64_t)n * ep.bias_stride] : 0.0f);
    if (ep.causal_mask && n > m) val = -INFINITY;
    C.p[zo * C.s_outer + zi * C.s_inner + (int64_t)m * C.s_row + n] = val;
  }
}

bool vec_ok(const GemmOperand& op, bool contig_is_col) {
  // dwordx4 loads along the contiguous dimension need 16-byte aligned rows.
  const int64_t s_other = contig_is_col ? op.s_row : op.s_col;
  return aligned16(op.p) && s_other % 4 == 0 && op.s_outer % 4 == 0 && op.s_inner % 4 == 0;
}

int pick_mode(const GemmOperand& op, bool is_a) {
  // For A: (s_row, s_col) = (m, k) -> kVecK when k is contiguous.
  // For B: (s_row, s_col) = (k, n) -> kVecK (n-major, k contiguous) when s_row == 1.
  const int64_t s_k = is_a ? op.s_col : op.s_row;
  const int64_t s_mn = is_a ? op.s_row : op.s_col;
  if (s_k == 1 && vec_ok(op, is_a)) return kVecK;
  if (s_mn == 1 && vec_ok(op, !is_a)) return kVecMN;
  return kScalar;
}

template <int AM>
void dispatch_b(int bm, dim3 grid, hipStream_t st, const GemmOperand& A, const GemmOperand& B,
                const GemmOut& C, const GemmEpilogue& ep, int M, int N, int K, int zin, int Z,
                int kchunk, float* ws) {
  if (bm == kVecK)
    hipLaunchKernelGGL((gemm_kernel<AM, kVecK>), grid, dim3(256), 0, st, A, B, C, ep, M, N, K, zin,
                       Z, kchunk, ws);
  else if (bm == kVecMN)
    hipLaunchKernelGGL((gemm_kernel<AM, kVecMN>), grid, dim3(256), 0, st, A, B, C, ep, M, N, K,
                       zin, Z, kchunk, ws);
  else
    hipLaunchKernelGGL((gemm_kernel<AM, kScalar>), grid, dim3(256), 0, st, A, B, C, ep, M, N, K,
                       zin, Z, kchunk, ws);
}

// K splits for a GEMM whose output tiles alone cannot fill the 256 CUs: enough splits for
// ~512 workgroups, each keeping at least 512 of K; 1 = no split.
int64_t splitk_factor(int64_t M, int64_t N, int64_t K, int64_t Z) {
  const int64_t tiles = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN) * Z;
  if (tiles >= 256 || K < 1024) return 1;
  const int64_t s = std::min<int64_t>({(512 + tiles - 1) / tiles, K / 512, 8});
  return s >= 2 ? s : 1;
}

}  // namespace

int64_t gemm_workspace_floats(int64_t M, int64_t N, int64_t K, int64_t Z) {
  const int64_t S = splitk_factor(M, N, K, Z);
  return S > 1 ? S * Z * M * N : 0;
}

// Launch the strided batched GEMM.  Z = number of batches, zin = inner batch extent.  With a
// workspace of gemm_workspace_floats() floats, low-parallelism shapes are split along K.
int gemm_launch(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z, int64_t zin,
                hipStream_t st, float* workspace, int64_t workspace_floats) {
  if (M <= 0 || N <= 0 || Z <= 0) return CTA_OK;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || Z > 65535 || zin <= 0)
    return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM size out of range");
  int64_t S = splitk_factor(M, N, K, Z);
  if (S > 1 && (workspace == nullptr || workspace_floats < S * Z * M * N)) S = 1;
  const int64_t kchunk = S > 1 ? ((K + S - 1) / S + GBK - 1) / GBK * GBK : std::max<int64_t>(K, 1);
  const dim3 grid((unsigned)((N + GBN - 1) / GBN), (unsigned)((M + GBM - 1) / GBM),
                  (unsigned)(Z * S));
  if (grid.y > 65535 || grid.z > 65535) return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM grid too large");
  float* ws = S > 1 ? workspace : nullptr;
  const int am = pick_mode(A, true);
  const int bm = pick_mode(B, false);
  if (am == kVecK)
    dispatch_b<kVecK>(bm, grid, st, A, B, C, ep, (int)M, (int)N, (int)K, (int)zin, (int)Z, (int)kchunk, ws);
  else if (am == kVecMN)
    dispatch_b<kVecMN>(bm, grid, st, A, B, C, ep, (int)M, (int)N, (int)K, (int)zin, (int)Z, (int)kchunk, ws);
  else
    dispatch_b<kScalar>(bm, grid, st, A, B, C, ep, (int)M, (int)N, (int)K, (int)zin, (int)Z, (int)kchunk, ws);
  if (S > 1) {
    const int64_t total = Z * M * N;
    const unsigned rgrid = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(rgrid), dim3(256), 0, st, ws, (int)S, (int)Z,
                       (int)M, (int)N, C, ep, (int)zin);
  }
  return check_launch("gemm");
}

}  // namespace cta

using namespace cta;

extern "C" int64_t cta_cuda_fma_workspace(int64_t batch, int64_t m, int64_t k, int64_t n) {
  if (batch <= 0 || m <= 0 || n <= 0 || k <= 0) return 0;
  return gemm_workspace_floats(m, n, k, batch) * (int64_t)sizeof(float);
}

extern "C" int cta_cuda_fma(const float* x, const int64_t* x_strides, const float* w,
                            const int64_t* w_strides, const float* bias, int64_t bias_stride,
                            int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                            float* out, float* workspace, void* stream) {
  if (batch < 0 || m < 0 || k < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (w_batch != 1 && w_batch != batch)
    return fail(CTA_ERR_INVALID_ARGUMENT, "weights batch must be 1 or equal to x batch");
  if (batch * m * n == 0) return CTA_OK;
  if (!x || !w || !bias || !out || !x_strides || !w_strides)
    return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  const GemmOperand A{x, x_strides[0], 0, x_strides[1], x_strides[2]};
  // Broadcast weights use batch stride 0, as linear_layer.cu:30-34 does.
  const GemmOperand B{w, w_batch == 1 ? 0 : w_strides[0], 0, w_strides[1], w_strides[2]};
  const GemmOut C{out, m * n, 0, n};
  const GemmEpilogue ep{1.0f, bias, bias_stride, 0};
  return gemm_launch(A, B, C, ep, m, n, k, batch, 1, as_stream(stream), workspace,
                     workspace ? gemm_workspace_floats(m, n, k, batch) : 0);
}

extern "C" int64_t cta_db_calculation_workspace(int64_t batch, int64_t m, int64_t n) {
  if (batch <= 0 || m <= 0 || n <= 0) return 0;
  return colsum_chunks(batch * m) * n * (int64_t)sizeof(float);
}

extern "C" int cta_db_calculation(const float* dy, const int64_t* dy_strides, int64_t batch,
                                  int64_t m, int64_t n, float* db, float* workspace,
                                  void* stream) {
  if (batch < 0 || m < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (n == 0) return CTA_OK;
  if (!db) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  hipStream_t st = as_stream(stream);
  if (batch * m == 0) {
    if (hipMemsetAsync(db, 0, n * sizeof(float), st) != hipSuccess)
      return fail(CTA_ERR_LAUNCH, "hipMemsetAsync failed");
    return CTA_OK;
  }
  if (!dy || !dy_strides || !workspace) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  return colsum_launch(dy, batch, m, n, dy_strides[0], dy_strides[1], dy_strides[2], db,
                       workspace, st);
}
