// Deterministic column reductions (no atomics) on gfx950.
//
//  * colsum_rows: per-chunk column sums of a strided (batch, m, n) tensor — the first stage of
//    the bias gradient db[n] = sum over (batch, m) of dy (the reference reduces one column per
//    1024-thread block with strided reads: warp_sum_kernel.cuh:13-51).  Each thread owns 4
//    adjacent columns (dwordx4) or 1 column, walks 32 rows of its chunk eight at a time into
//    eight independent accumulators, and writes one partial row.  Row pointers advance incrementally, so there is
//    no division in the loop.
//  * colsum_partials: sums a [chunks][ncols] partial matrix over its rows in a fixed order, so
//    results are bitwise reproducible.  With float4-aligned columns, in one launch (16 row
//    phases per float4 column group, combined in LDS).  Otherwise, given scratch, in two stages:
//    up to 16 row groups of 64-column blocks in parallel (four row phases per column, combined
//    in LDS), then one pass over the group sums; without scratch, one workgroup per 32 columns
//    walks every row.
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
  // eight rows in flight per thread, each into its own accumulator
  float4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = zero4();
  auto load = [&](const float* q) -> float4 {
    if (VEC) return ld4(q);
    return make_float4(q[0], 0.f, 0.f, 0.f);
  };
  int64_t r = r0;
  for (; r + 8 <= r1; r += 8) {
    const float* q[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      q[u] = p;
      advance();
    }
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = load(q[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc[u].x += v[u].x; acc[u].y += v[u].y; acc[u].z += v[u].z; acc[u].w += v[u].w;
    }
  }
#pragma unroll
  for (int u = 0; u < 7; ++u) {  // the last r1 - r < 8 rows; u stays a constant per copy
    if (r + u < r1) {
      const float4 v = load(p);
      advance();
      acc[u].x += v.x; acc[u].y += v.y; acc[u].z += v.z; acc[u].w += v.w;
    }
  }
  auto sum8 = [&](auto get) {
    return ((get(acc[0]) + get(acc[1])) + (get(acc[2]) + get(acc[3]))) +
           ((get(acc[4]) + get(acc[5])) + (get(acc[6]) + get(acc[7])));
  };
  const float4 s = make_float4(sum8([](float4 a) { return a.x; }), sum8([](float4 a) { return a.y; }),
                               sum8([](float4 a) { return a.z; }), sum8([](float4 a) { return a.w; }));
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

// One-launch sum of a [chunks][ncols] partial matrix when ncols and the split are multiples of
// 4 and every buffer is 16-byte aligned: a workgroup owns 16 float4 column groups, and its 16
// row phases each add every 16th partial row in row order, 16 rows at a time with all 16 loads
// in flight (addresses clamped to the last row, rows past it selected away, so the loads are
// branch-free); then phase 0 adds the 16 phase sums in order.  Fixed order throughout: bitwise
// reproducible.
constexpr int kWideCols4 = 16;
constexpr int kWidePhases = 16;
constexpr int kWideBatch = 16;

__global__ __launch_bounds__(kWideCols4 * kWidePhases) void colsum_wide_kernel(
    const float* __restrict__ part, int64_t chunks, int64_t ncols, float* __restrict__ out0,
    float* __restrict__ out1, int64_t split) {
  __shared__ float4 red[kWidePhases][kWideCols4];
  const int c4 = threadIdx.x % kWideCols4, ph = threadIdx.x / kWideCols4;
  const int64_t col = ((int64_t)blockIdx.x * kWideCols4 + c4) * 4;
  float4 acc = zero4();
  if (col < ncols) {
    for (int64_t base = ph; base < chunks; base += kWidePhases * kWideBatch) {
      float4 v[kWideBatch];
#pragma unroll
      for (int u = 0; u < kWideBatch; ++u)
        v[u] = ld4(part + min(base + u * kWidePhases, chunks - 1) * ncols + col);
#pragma unroll
      for (int u = 0; u < kWideBatch; ++u) {
        if (base + u * kWidePhases < chunks) {
          acc.x += v[u].x; acc.y += v[u].y; acc.z += v[u].z; acc.w += v[u].w;
        }
      }
    }
  }
  red[ph][c4] = acc;
  __syncthreads();
  if (ph == 0 && col < ncols) {
    float4 t = red[0][c4];
#pragma unroll
    for (int p = 1; p < kWidePhases; ++p) {
      t.x += red[p][c4].x; t.y += red[p][c4].y; t.z += red[p][c4].z; t.w += red[p][c4].w;
    }
    if (col < split) st4(out0 + col, t);
    else st4(out1 + (col - split), t);
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
  if (ncols % 4 == 0 && split % 4 == 0 && aligned16(part) && aligned16(out0) &&
      aligned16(out1)) {
    const unsigned grid = (unsigned)((ncols / 4 + kWideCols4 - 1) / kWideCols4);
    hipLaunchKernelGGL(colsum_wide_kernel, dim3(grid), dim3(kWideCols4 * kWidePhases), 0, st,
                       part, chunks, ncols, out0, out1, split);
    return check_launch("column sum");
  }
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
