// Deterministic column reductions (no atomics) on gfx950.
//
//  * colsum_rows: per-chunk column sums of a strided (batch, m, n) tensor — the first stage of
//    the bias gradient db[n] = sum over (batch, m) of dy (the reference reduces one column per
//    1024-thread block with strided reads: warp_sum_kernel.cuh:13-51).  Each thread owns 4
//    adjacent columns (dwordx4) or 1 column, walks 32 rows of its chunk with four independent
//    accumulators, and writes one partial row.  Row pointers advance incrementally, so there is
//    no division in the loop.
//  * colsum_partials: sums a [chunks][ncols] partial matrix over its rows in a fixed order, so
//    results are bitwise reproducible.  Given scratch, in two stages: up to 16 row groups of
//    64-column blocks in parallel (four row phases per column, combined in LDS), then one pass
//    over the group sums; without scratch, one workgroup per 32 columns walks every row.
#include "cta_common.hpp"
#include "gemm.hpp"

namespace cta {
namespace {

constexpr int kRowsPerChunk = 32;
constexpr int kTreeCols = 32;    // columns per workgroup in the final sum
constexpr int kTreeGroups = 8;   // row groups per column

template <bool VEC>
__global__ __launch_bounds__(256) void colsum_rows_kernel(const float* __restrict__ x,
                                                          float* __restrict__ part, int64_t M,
                                                          int64_t N, int64_t sb, int64_t sm,
                                                          int64_t sn, int64_t rows, int rpc) {
  constexpr int W = VEC ? 4 : 1;
  const int64_t col0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * W;
  if (col0 >= N) return;
  const int64_t r0 = (int64_t)blockIdx.y * rpc;
  const int64_t r1 = min(rows, r0 + rpc);
  int64_t b = r0 / M, m = r0 - b * M;
  const float* p = x + b * sb + m * sm + col0 * sn;
  auto advance = [&]() {
    p += sm;
    if (++m == M) {
      m = 0;
      ++b;
      p = x + b * sb + col0 * sn;
    }
  };
  float4 acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) acc[u] = zero4();
  auto load = [&](const float* q) -> float4 {
    if (VEC) return ld4(q);
    return make_float4(q[0], 0.f, 0.f, 0.f);
  };
  int64_t r = r0;
  for (; r + 4 <= r1; r += 4) {
    const float* q0 = p; advance();
    const float* q1 = p; advance();
    const float* q2 = p; advance();
    const float* q3 = p; advance();
    const float4 v0 = load(q0), v1 = load(q1), v2 = load(q2), v3 = load(q3);
    acc[0].x += v0.x; acc[0].y += v0.y; acc[0].z += v0.z; acc[0].w += v0.w;
    acc[1].x += v1.x; acc[1].y += v1.y; acc[1].z += v1.z; acc[1].w += v1.w;
    acc[2].x += v2.x; acc[2].y += v2.y; acc[2].z += v2.z; acc[2].w += v2.w;
    acc[3].x += v3.x; acc[3].y += v3.y; acc[3].z += v3.z; acc[3].w += v3.w;
  }
  for (; r < r1; ++r) {
    const float4 v = load(p);
    advance();
    acc[0].x += v.x; acc[0].y += v.y; acc[0].z += v.z; acc[0].w += v.w;
  }
  const float4 s = make_float4((acc[0].x + acc[1].x) + (acc[2].x + acc[3].x),
                               (acc[0].y + acc[1].y) + (acc[2].y + acc[3].y),
                               (acc[0].z + acc[1].z) + (acc[2].z + acc[3].z),
                               (acc[0].w + acc[1].w) + (acc[2].w + acc[3].w));
  float* out = part + (int64_t)blockIdx.y * N + col0;
  if (VEC) st4(out, s);
  else out[0] = s.x;
}

__global__ __launch_bounds__(256) void colsum_tree_kernel(const float* __restrict__ part,
                                                          int64_t chunks, int64_t ncols,
                                                          float* __restrict__ out0,
                                                          float* __restrict__ out1,
                                                          int64_t split) {
  __shared__ float red[kTreeGroups][kTreeCols];
  const int c = threadIdx.x % kTreeCols, g = threadIdx.x / kTreeCols;
  const int64_t col = (int64_t)blockIdx.x * kTreeCols + c;
  float a0 = 0.f, a1 = 0.f;
  if (col < ncols) {
    int64_t k = g;
    for (; k + kTreeGroups < chunks; k += 2 * kTreeGroups) {
      a0 += part[k * ncols + col];
      a1 += part[(k + kTreeGroups) * ncols + col];
    }
    if (k < chunks) a0 += part[k * ncols + col];
  }
  red[g][c] = a0 + a1;
  __syncthreads();
  if (g == 0 && col < ncols) {
    float s = red[0][c];
#pragma unroll
    for (int i = 1; i < kTreeGroups; ++i) s += red[i][c];
    if (col < split) out0[col] = s;
    else out1[col - split] = s;
  }
}

constexpr int kGroupCols = 64;      // columns per workgroup in the grouped first stage
constexpr int kGroupPhases = 4;     // row phases per column (256 threads = 64 x 4)
constexpr int kRowsPerGroup = 32;   // target rows per group
constexpr int kMaxGroups = 16;

// Stage 1: group g of rows [g*rpg, min(chunks, (g+1)*rpg)) for 64 columns -> scratch[g][col].
__global__ __launch_bounds__(256) void colsum_group_kernel(const float* __restrict__ part,
                                                           int64_t chunks, int64_t ncols,
                                                           int64_t rpg,
                                                           float* __restrict__ scratch) {
  __shared__ float red[kGroupPhases][kGroupCols];
  const int c = threadIdx.x % kGroupCols, ph = threadIdx.x / kGroupCols;
  const int64_t col = (int64_t)blockIdx.x * kGroupCols + c;
  const int64_t r0 = (int64_t)blockIdx.y * rpg, r1 = min(chunks, r0 + rpg);
  float a0 = 0.f, a1 = 0.f;
  if (col < ncols) {
    int64_t r = r0 + ph;
    for (; r + kGroupPhases < r1; r += 2 * kGroupPhases) {
      a0 += part[r * ncols + col];
      a1 += part[(r + kGroupPhases) * ncols + col];
    }
    if (r < r1) a0 += part[r * ncols + col];
  }
  red[ph][c] = a0 + a1;
  __syncthreads();
  if (ph == 0 && col < ncols)
    scratch[(int64_t)blockIdx.y * ncols + col] = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
}

// Stage 2: out[col] = sum over the group sums: each of four phases adds every fourth group in
// order, then the phases are combined in order.
__global__ __launch_bounds__(256) void colsum_final_kernel(const float* __restrict__ scratch,
                                                           int groups, int64_t ncols,
                                                           float* __restrict__ out0,
                                                           float* __restrict__ out1,
                                                           int64_t split) {
  __shared__ float red[kGroupPhases][kGroupCols];
  const int c = threadIdx.x % kGroupCols, ph = threadIdx.x / kGroupCols;
  const int64_t col = (int64_t)blockIdx.x * kGroupCols + c;
  float a = 0.f;
  if (col < ncols)
    for (int g = ph; g < groups; g += kGroupPhases) a += scratch[(int64_t)g * ncols + col];
  red[ph][c] = a;
  __syncthreads();
  if (ph == 0 && col < ncols) {
    const float s = (red[0][c] + red[1][c]) + (red[2][c] + red[3][c]);
    if (col < split) out0[col] = s;
    else out1[col - split] = s;
  }
}

int64_t rows_per_chunk(int64_t rows) {
  return std::max<int64_t>(kRowsPerChunk, (rows + 65534) / 65535);
}

int64_t colsum_groups(int64_t chunks) {
  return std::min<int64_t>(kMaxGroups, std::max<int64_t>(1, (chunks + kRowsPerGroup - 1) / kRowsPerGroup));
}

}  // namespace

int64_t colsum_partials_scratch_floats(int64_t chunks, int64_t ncols) {
  return colsum_groups(chunks) * ncols;
}

int colsum_partials_launch(const float* part, int64_t chunks, int64_t ncols, float* out0,
                           float* out1, int64_t split, hipStream_t st, float* scratch) {
  if (scratch == nullptr) {
    const unsigned grid = (unsigned)((ncols + kTreeCols - 1) / kTreeCols);
    hipLaunchKernelGGL(colsum_tree_kernel, dim3(grid), dim3(256), 0, st, part, chunks, ncols,
                       out0, out1, split);
    return check_launch("column sum");
  }
  const int64_t groups = colsum_groups(chunks);
  const int64_t rpg = (chunks + groups - 1) / groups;
  hipLaunchKernelGGL(colsum_group_kernel,
                     dim3((unsigned)((ncols + kGroupCols - 1) / kGroupCols), (unsigned)groups),
                     dim3(256), 0, st, part, chunks, ncols, rpg, scratch);
  hipLaunchKernelGGL(colsum_final_kernel, dim3((unsigned)((ncols + kGroupCols - 1) / kGroupCols)),
                     dim3(256), 0, st, scratch, (int)groups, ncols, out0, out1, split);
  return check_launch("column sum");
}

int64_t colsum_chunks(int64_t rows) {
  return rows <= 0 ? 0 : (rows + rows_per_chunk(rows) - 1) / rows_per_chunk(rows);
}

int64_t colsum_workspace_floats(int64_t rows, int64_t N) {
  const int64_t chunks = colsum_chunks(rows);
  return chunks * N + colsum_partials_scratch_floats(chunks, N);
}

int colsum_launch(const float* x, int64_t batch, int64_t M, int64_t N, int64_t sb, int64_t sm,
                  int64_t sn, float* out, float* workspace, hipStream_t st) {
  const int64_t rows = batch * M;
  const int64_t rpc = rows_per_chunk(rows);
  const int64_t chunks = colsum_chunks(rows);
  if (chunks > 65535 || N > INT32_MAX) return fail(CTA_ERR_INVALID_ARGUMENT, "column sum too large");
  if (batch == 1) sb = 0;  // the batch stride of a single batch is never used
  const bool vec = sn == 1 && N % 4 == 0 && aligned16(x) && sm % 4 == 0 && sb % 4 == 0;
  const int64_t per_block = vec ? 1024 : 256;
  const dim3 grid((unsigned)((N + per_block - 1) / per_block), (unsigned)chunks);
  if (vec)
    hipLaunchKernelGGL((colsum_rows_kernel<true>), grid, dim3(256), 0, st, x, workspace, M, N, sb,
                       sm, sn, rows, (int)rpc);
  else
    hipLaunchKernelGGL((colsum_rows_kernel<false>), grid, dim3(256), 0, st, x, workspace, M, N, sb,
                       sm, sn, rows, (int)rpc);
  if (int rc = check_launch("db_calculation")) return rc;
  return colsum_partials_launch(workspace, chunks, N, out, out, N, st, workspace + chunks * N);
}

}  // namespace cta
