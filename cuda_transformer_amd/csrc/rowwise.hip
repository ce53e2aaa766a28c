// Bandwidth-bound kernels: exact GELU, row softmax, LayerNorm (forward and backward), and a
// tanh-approximated GELU.
//
//  * GELU follows Transformer_kernels/GeLU.cuh:7-29: y = x Phi(x),
//    dx = dy (Phi(x) + x phi(x)), phi(x) = e^{-x^2/2} / sqrt(2 pi); Phi from a Chebyshev-fitted
//    erfc (cta_common.hpp), short enough that the kernels stay HBM-bound.
//  * The tanh GELU has no reference kernel; it is torch's F.gelu(x, approximate="tanh").
//  * Softmax follows softmax.cuh:25-159 (row max, sum of e^{x - max}, normalise;
//    backward dx = p (dp - sum p dp)).
//  * LayerNorm has no kernel in the reference; its semantics come from gpt/gpt.py:47-59:
//    y = (x - mean) / sqrt(var + eps) * gamma + beta with the biased variance.
//
// gfx950 design: HBM is the bound, so every kernel moves each byte once.  Elementwise kernels
// use dwordx4 loads/stores.  Row kernels give one wave64 to one row, keep the whole row in
// registers (up to 2048 columns) and reduce with cross-lane shuffles — a single read and a
// single write per element, where the reference reads x three times.  Longer rows fall back
// to a workgroup-per-row path.  Column reductions (dgamma, dbeta) are two-stage and
// deterministic (no atomics).
#include "cta_common.hpp"
#include "gemm.hpp"

namespace cta {
namespace {

// ------------------------------------------------------------------------------- GELU
// (gelu_f / gelu_grad and gelu_tanh_f / gelu_tanh_grad live in cta_common.hpp, shared with the
// GEMM epilogue.)

template <bool TANH>
__device__ __forceinline__ float gelu_act(float x) {
  return TANH ? gelu_tanh_f(x) : gelu_f(x);
}
template <bool TANH>
__device__ __forceinline__ float gelu_act_grad(float x, float g) {
  return TANH ? gelu_tanh_grad(x, g) : gelu_grad(x, g);
}

// Each thread handles four independent float4 per iteration (index i + 256*u within a chunk of
// 1024 float4) so that four loads are in flight before the math starts.
template <bool TANH>
__device__ __forceinline__ void gelu_fwd_body(const float* __restrict__ x, float* __restrict__ y,
                                              int64_t n4, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 1024;
  for (int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x; base < n4; base += stride) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + 256 * u;
      v[u] = (i < n4) ? ld4(x + 4 * i) : zero4();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + 256 * u;
      if (i < n4)
        st4(y + 4 * i, make_float4(gelu_act<TANH>(v[u].x), gelu_act<TANH>(v[u].y),
                                   gelu_act<TANH>(v[u].z), gelu_act<TANH>(v[u].w)));
    }
  }
  // tail (n % 4 elements) handled by the first threads of block 0
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
    const int64_t i = 4 * n4 + threadIdx.x;
    y[i] = gelu_act<TANH>(x[i]);
  }
}

template <bool TANH>
__device__ __forceinline__ void gelu_bwd_body(const float* __restrict__ x,
                                              const float* __restrict__ dy,
                                              float* __restrict__ dx, int64_t n4, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 1024;
  for (int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x; base < n4; base += stride) {
    float4 v[4], g[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + 256 * u;
      v[u] = (i < n4) ? ld4(x + 4 * i) : zero4();
      g[u] = (i < n4) ? ld4(dy + 4 * i) : zero4();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + 256 * u;
      if (i < n4)
        st4(dx + 4 * i,
            make_float4(gelu_act_grad<TANH>(v[u].x, g[u].x), gelu_act_grad<TANH>(v[u].y, g[u].y),
                        gelu_act_grad<TANH>(v[u].z, g[u].z), gelu_act_grad<TANH>(v[u].w, g[u].w)));
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) {
    const int64_t i = 4 * n4 + threadIdx.x;
    dx[i] = gelu_act_grad<TANH>(x[i], dy[i]);
  }
}

// One kernel name per form, so that kernel traces tell them apart.
__global__ __launch_bounds__(256) void gelu_fwd_kernel(const float* __restrict__ x,
                                                       float* __restrict__ y, int64_t n4,
                                                       int64_t n) {
  gelu_fwd_body<false>(x, y, n4, n);
}
__global__ __launch_bounds__(256) void gelu_bwd_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ dy,
                                                       float* __restrict__ dx, int64_t n4,
                                                       int64_t n) {
  gelu_bwd_body<false>(x, dy, dx, n4, n);
}
__global__ __launch_bounds__(256) void gelu_tanh_fwd_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t n4,
                                                            int64_t n) {
  gelu_fwd_body<true>(x, y, n4, n);
}
__global__ __launch_bounds__(256) void gelu_tanh_bwd_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ dy,
                                                            float* __restrict__ dx, int64_t n4,
                                                            int64_t n) {
  gelu_bwd_body<true>(x, dy, dx, n4, n);
}

unsigned elementwise_grid(int64_t n4) {
  // enough workgroups to fill 256 CUs several times over; grid-stride covers the rest
  const int64_t want = (n4 + 1023) / 1024;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 256 * 16));
}

// Plain dwordx4 copy, four float4 per thread in flight per iteration (the elementwise kernels'
// access pattern without their arithmetic): the streaming ceiling of a read + write pass.
__global__ __launch_bounds__(256) void device_copy_kernel(const float* __restrict__ src,
                                                          float* __restrict__ dst, int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * 1024;
  for (int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x; base < n4; base += stride) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + 256 * u;
      v[u] = (i < n4) ? ld4(src + 4 * i) : zero4();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t i = base + 256 * u;
      if (i < n4) st4(dst + 4 * i, v[u]);
    }
  }
}

__global__ __launch_bounds__(256) void zero_fill_kernel(float* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    p[i] = 0.0f;
}

// ------------------------------------------------------------------- row register path
// A wave owns one row of length n.  VEC: n % 4 == 0 and rows 16-byte aligned, lane loads
// float4 chunks c = lane + 64*u; otherwise lane loads scalars e = lane + 64*u.
template <int U, bool VEC>
struct RowRegs {
  static constexpr int W = VEC ? 4 : 1;
  float v[U * W];
  // STREAM: the non-temporal forms (rows read or written once, in passes larger than the
  // caches)
  template <bool STREAM = false>
  __device__ __forceinline__ void load(const float* row, int n, int lane, float fill) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = lane + 64 * u;
      if (VEC) {
        const float4 t = (4 * c < n) ? (STREAM ? ld4_stream(row + 4 * c) : ld4(row + 4 * c))
                                     : make_float4(fill, fill, fill, fill);
        v[4 * u + 0] = t.x; v[4 * u + 1] = t.y; v[4 * u + 2] = t.z; v[4 * u + 3] = t.w;
      } else {
        v[u] = (c < n) ? row[c] : fill;
      }
    }
  }
  template <bool STREAM = false>
  __device__ __forceinline__ void store(float* row, int n, int lane) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = lane + 64 * u;
      if (VEC) {
        if (4 * c < n) {
          const float4 t = make_float4(v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]);
          if (STREAM)
            st4_stream(row + 4 * c, t);
          else
            st4(row + 4 * c, t);
        }
      } else {
        if (c < n) row[c] = v[u];
      }
    }
  }
  // column index of element e of this lane
  __device__ __forceinline__ static int colof(int e, int lane) {
    return VEC ? 4 * (lane + 64 * (e / 4)) + (e % 4) : lane + 64 * e;
  }
};

// Softmax rows: one wave per row, the whole row in registers.  The grid covers every row up
// to 2^22 rows; beyond that each wave strides on by 4 gridDim.x rows.  (Several rows per wave
// with the next row prefetched measured 5% slower at 48K rows of 1024: fewer waves in flight.)
// x and y (p, dp and dx) may be the same buffer: a wave reads its row completely before it
// writes it.  Rows are read and written with the non-temporal bit: config 4's softmax moves
// 400-600 MB per pass, more than the 256 MB MALL, and the streaming forms measured forward
// 71.3 -> 65.4 us and backward 106.4 -> 92.0 us cache-cold (48K rows of 1024).
template <int U, bool VEC>
__global__ __launch_bounds__(256) void softmax_fwd_rows(const float* x, float* y, int64_t rows,
                                                        int n) {
  const int lane = threadIdx.x & 63;
  const int64_t step = (int64_t)gridDim.x * 4;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave_index(); row < rows; row += step) {
    RowRegs<U, VEC> r;
    r.template load<true>(x + row * n, n, lane, -INFINITY);
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < U * r.W; ++e) mx = fmaxf(mx, r.v[e]);
    mx = wave_max(mx);
    // e^{v - mx} = 2^{(v - mx) log2(e)} with the hardware exp2.  The difference is taken
    // first: folding mx log2(e) into one rounded offset would leave that rounding error
    // (up to 2^-25 |mx log2(e)|, about 440 at |mx| = 1e10) in every exponent, and overflow
    // to inf for |mx| above 2.36e38.  The row max then gets exactly 2^0 at any magnitude.
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < U * r.W; ++e) {
      const float p = __builtin_amdgcn_exp2f((r.v[e] - mx) * kLog2e);
      r.v[e] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int e = 0; e < U * r.W; ++e) r.v[e] *= inv;
    r.template store<true>(y + row * n, n, lane);
  }
}

template <int U, bool VEC>
__global__ __launch_bounds__(256) void softmax_bwd_rows(const float* p, const float* dp,
                                                        float* dx, int64_t rows, int n) {
  const int lane = threadIdx.x & 63;
  const int64_t step = (int64_t)gridDim.x * 4;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave_index(); row < rows; row += step) {
    RowRegs<U, VEC> a, g;
    a.template load<true>(p + row * n, n, lane, 0.0f);
    g.template load<true>(dp + row * n, n, lane, 0.0f);
    float dot = 0.0f;
#pragma unroll
    for (int e = 0; e < U * a.W; ++e) dot = fmaf(a.v[e], g.v[e], dot);
    dot = wave_sum(dot);
#pragma unroll
    for (int e = 0; e < U * a.W; ++e) a.v[e] = a.v[e] * (g.v[e] - dot);
    a.template store<true>(dx + row * n, n, lane);
  }
}

// --------------------------------------------------------------- long-row block path
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // red[] may still be read by a previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

__global__ __launch_bounds__(256) void softmax_fwd_long(const float* x, float* y,
                                                        int64_t rows, int n) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float* xr = x + row * n;
    float* yr = y + row * n;
    // pass 1: online max/sum per thread, then a block-wide merge of the (max, sum) pairs
    float m = -INFINITY, s = 0.0f;
    for (int c = threadIdx.x; c < n; c += 256) {
      const float v = xr[c];
      const float mn = fmaxf(m, v);
      if (mn != -INFINITY) {  // masked (-inf) entries before the first finite one add nothing
        s = s * expf(m - mn) + expf(v - mn);
        m = mn;
      }
    }
    const float gm = block_reduce(m, true, red);
    const float part = (m == -INFINITY) ? 0.0f : s * expf(m - gm);
    const float gs = block_reduce(part, false, red);
    const float inv = 1.0f / gs;
    for (int c = threadIdx.x; c < n; c += 256) yr[c] = expf(xr[c] - gm) * inv;
  }
}

__global__ __launch_bounds__(256) void softmax_bwd_long(const float* p, const float* dp,
                                                        float* dx, int64_t rows, int n) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float* pr = p + row * n;
    const float* gr = dp + row * n;
    float* xr = dx + row * n;
    float dot = 0.0f;
    for (int c = threadIdx.x; c < n; c += 256) dot = fmaf(pr[c], gr[c], dot);
    dot = block_reduce(dot, false, red);
    __syncthreads();  // every thread has read its p/dp before any in-place write lands
    for (int c = threadIdx.x; c < n; c += 256) xr[c] = pr[c] * (gr[c] - dot);
  }
}

// ------------------------------------------------------------------------ LayerNorm
// a + b rounded once and never fused with the multiply that produced a, so that the residual
// variants below give the bits of a separate LayerNorm kernel followed by an add.
__device__ __forceinline__ float add_unfused(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// RES: the row is x + f, stored to xsum before it is normalised (a residual add fused with the
// LayerNorm that follows it).
template <int U, bool VEC, bool RES = false>
__global__ __launch_bounds__(256) void layernorm_fwd_rows(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float* __restrict__ y, float* __restrict__ mean, float* __restrict__ rstd, int64_t rows,
    int n, float eps, const float* __restrict__ f = nullptr, float* __restrict__ xsum = nullptr) {
  const int lane = threadIdx.x & 63;
  const int64_t step = (int64_t)gridDim.x * 4;
  for (int64_t row = (int64_t)blockIdx.x * 4 + wave_index(); row < rows; row += step) {
    using R = RowRegs<U, VEC>;
    R r, gm, bt;
    r.load(x + row * n, n, lane, 0.0f);
    if constexpr (RES) {
      R fr;
      fr.load(f + row * n, n, lane, 0.0f);
#pragma unroll
      for (int e = 0; e < U * R::W; ++e) r.v[e] += fr.v[e];
      r.store(xsum + row * n, n, lane);
    }
    gm.load(gamma, n, lane, 0.0f);
    bt.load(beta, n, lane, 0.0f);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < U * R::W; ++e) s += r.v[e];
    const float mu = wave_sum(s) / (float)n;
    float q = 0.0f;
#pragma unroll
    for (int e = 0; e < U * R::W; ++e) {
      const float d = (R::colof(e, lane) < n) ? r.v[e] - mu : 0.0f;
      q = fmaf(d, d, q);
    }
    const float var = wave_sum(q) / (float)n;
    const float rs = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int e = 0; e < U * R::W; ++e) r.v[e] = fmaf((r.v[e] - mu) * rs, gm.v[e], bt.v[e]);
    r.store(y + row * n, n, lane);
    if (lane == 0) {
      mean[row] = mu;
      rstd[row] = rs;
    }
  }
}

// Backward: WAVES waves per workgroup (16 when a row takes at most 12 registers per lane, so
// that 16 waves fit 128 VGPRs each; 8 otherwise).  Each wave takes its rows two at a time (one
// at a time for rows above 16 registers per lane), both rows' loads in flight before either is
// reduced; dx stays in registers.  With one 16-wave workgroup per CU and two rows per wave, all
// 8192 rows of a GPT-2-small activation are in flight at once.  The waves' dgamma / dbeta
// column sums are combined in LDS by a fixed tree (waves 8-15 into 0-7, 4-7 into 0-3, 2-3 into
// 0-1, 1 into 0: bitwise reproducible) and written as one partial row per workgroup to `part`
// ([blocks][2][n]); colsum_partials then adds the partial rows in row order.  (Measured at
// 8192 x 768, event-timed: 19.2 us against 19.9 us for four-wave workgroups with the next row
// prefetched and 21.6 us for four-wave workgroups without.)
template <int U, bool VEC>
constexpr int ln_bwd_waves() {
  return U * RowRegs<U, VEC>::W <= 12 ? 16 : 8;
}

// RES: dx also receives dres, the gradient reaching the LayerNorm's input by the residual path.
template <int U, bool VEC, bool RES = false>
__global__ __launch_bounds__((64 * ln_bwd_waves<U, VEC>())) void layernorm_bwd_rows(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ dy, float* __restrict__ dx,
    float* __restrict__ part, int64_t rows, int n, int rows_per_wave,
    const float* __restrict__ dres = nullptr) {
  using R = RowRegs<U, VEC>;
  constexpr int E = U * R::W;
  constexpr int WAVES = ln_bwd_waves<U, VEC>();
  __shared__ float lds[WAVES / 2][2 * E * 64];
  const int lane = threadIdx.x & 63, wave = wave_index();
  R gm;
  gm.load(gamma, n, lane, 0.0f);
  float accg[E], accb[E];
#pragma unroll
  for (int e = 0; e < E; ++e) { accg[e] = 0.0f; accb[e] = 0.0f; }

  const int64_t r0 = ((int64_t)blockIdx.x * WAVES + wave) * rows_per_wave;
  const int64_t r1 = min(rows, r0 + rows_per_wave);
  const float inv_n = 1.0f / (float)n;
  auto row_grad = [&](R& xv, R& g, const R& dr, int64_t row) {
    const float mu = mean[row], rs = rstd[row];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float xh = (xv.v[e] - mu) * rs;
      const float gx = g.v[e] * gm.v[e];
      accg[e] = fmaf(g.v[e], xh, accg[e]);
      accb[e] += g.v[e];
      s1 += gx;
      s2 = fmaf(gx, xh, s2);
      xv.v[e] = xh;
      g.v[e] = gx;
    }
    const float m1 = wave_sum(s1) * inv_n, m2 = wave_sum(s2) * inv_n;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      xv.v[e] = rs * (g.v[e] - m1 - xv.v[e] * m2);
      if constexpr (RES) xv.v[e] = add_unfused(xv.v[e], dr.v[e]);
    }
    // dx with the non-temporal bit: 24.4 -> 22.9 us cache-cold at 8192 x 768, the GPT step
    // unchanged.  (The forward's y stays cached: a non-temporal y measured 14.8 -> 13.4 us alone
    // but cost the GPT step 0.3%, whose next GEMM reads y at once.)
    xv.template store<true>(dx + row * n, n, lane);
  };
  // two rows in flight while a row takes at most 16 registers per lane; one row beyond (two would
  // spill at 256 VGPRs)
  constexpr bool PAIR = E <= 16;
  for (int64_t a = r0; a < r1; a += PAIR ? 2 : 1) {
    const bool two = PAIR && a + 1 < r1;  // wave-uniform
    R xa, ga, xb, gb, ra, rb;
    xa.load(x + a * n, n, lane, 0.0f);
    ga.load(dy + a * n, n, lane, 0.0f);
    if (RES) ra.load(dres + a * n, n, lane, 0.0f);
    if (two) {
      xb.load(x + (a + 1) * n, n, lane, 0.0f);
      gb.load(dy + (a + 1) * n, n, lane, 0.0f);
      if (RES) rb.load(dres + (a + 1) * n, n, lane, 0.0f);
    }
    row_grad(xa, ga, ra, a);
    if (two) row_grad(xb, gb, rb, a + 1);
  }
  // fixed-order tree over the waves of this workgroup
#pragma unroll
  for (int half = WAVES / 2; half >= 1; half /= 2) {
    if (wave >= half && wave < 2 * half) {
      float* dst = lds[wave - half];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        dst[e * 64 + lane] = accg[e];
        dst[(E + e) * 64 + lane] = accb[e];
      }
    }
    __syncthreads();
    if (wave < half) {
      const float* src = lds[wave];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        accg[e] += src[e * 64 + lane];
        accb[e] += src[(E + e) * 64 + lane];
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int c = R::colof(e, lane);
      if (c < n) {
        part[(int64_t)blockIdx.x * 2 * n + c] = accg[e];
        part[(int64_t)blockIdx.x * 2 * n + n + c] = accb[e];
      }
    }
  }
}

// Long rows (n > 2048): one workgroup per row, three passes over the row.  With f the first
// pass forms x + f and stores it to xsum, and the later passes read xsum (each thread rereads
// the columns it wrote).
__global__ __launch_bounds__(256) void layernorm_fwd_long(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float* __restrict__ y, float* __restrict__ mean, float* __restrict__ rstd, int64_t rows,
    int n, float eps, const float* __restrict__ f, float* xsum) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float* xr = x + row * n;
    float s = 0.0f;
    if (f != nullptr) {
      float* sr = xsum + row * n;
      for (int c = threadIdx.x; c < n; c += 256) {
        const float v = xr[c] + f[row * n + c];
        sr[c] = v;
        s += v;
      }
      xr = sr;
    } else {
      for (int c = threadIdx.x; c < n; c += 256) s += xr[c];
    }
    const float mu = block_reduce(s, false, red) / (float)n;
    float q = 0.0f;
    for (int c = threadIdx.x; c < n; c += 256) {
      const float d = xr[c] - mu;
      q = fmaf(d, d, q);
    }
    const float rs = 1.0f / sqrtf(block_reduce(q, false, red) / (float)n + eps);
    for (int c = threadIdx.x; c < n; c += 256)
      y[row * n + c] = fmaf((xr[c] - mu) * rs, gamma[c], beta[c]);
    if (threadIdx.x == 0) {
      mean[row] = mu;
      rstd[row] = rs;
    }
  }
}

__global__ __launch_bounds__(256) void layernorm_bwd_long(
    const float* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ dy, float* __restrict__ dx,
    int64_t rows, int n, const float* __restrict__ dres) {
  __shared__ float red[4];
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const float mu = mean[row], rs = rstd[row];
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = threadIdx.x; c < n; c += 256) {
      const float xh = (x[row * n + c] - mu) * rs;
      const float gx = dy[row * n + c] * gamma[c];
      s1 += gx;
      s2 = fmaf(gx, xh, s2);
    }
    const float m1 = block_reduce(s1, false, red) / (float)n;
    const float m2 = block_reduce(s2, false, red) / (float)n;
    for (int c = threadIdx.x; c < n; c += 256) {
      const float xh = (x[row * n + c] - mu) * rs;
      const float gx = dy[row * n + c] * gamma[c];
      const float d = rs * (gx - m1 - xh * m2);
      dx[row * n + c] = dres ? add_unfused(d, dres[row * n + c]) : d;
    }
  }
}

// dgamma/dbeta for the long-row path: column partials over row chunks, then the final sum.
__global__ __launch_bounds__(256) void layernorm_colpart_long(
    const float* __restrict__ x, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ dy, float* __restrict__ part, int64_t rows, int n,
    int rows_per_block) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= n) return;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r1 = min(rows, r0 + rows_per_block);
  float sg = 0.0f, sb = 0.0f;
  for (int64_t r = r0; r < r1; ++r) {
    const float g = dy[r * n + c];
    sg = fmaf(g, (x[r * n + c] - mean[r]) * rstd[r], sg);
    sb += g;
  }
  part[(int64_t)blockIdx.y * 2 * n + c] = sg;
  part[(int64_t)blockIdx.y * 2 * n + n + c] = sb;
}

// ------------------------------------------------------------------ dispatch helpers
constexpr int kMaxRegCols = 2048;
constexpr int kLnBwdMaxBlocks = 256;  // partial rows for dgamma/dbeta (row-register path): one
                                      // 8- or 16-wave workgroup per CU
constexpr int kLnLongRowsPerBlock = 64;

// Register units per lane for a row of n columns: float4 units cover 256 columns each (3 and
// 6 fit the 768- and 1536-wide rows of GPT-style models exactly), scalar units 64.
int units_for(int n, bool vec) {
  const int per = vec ? 256 : 64;  // columns covered per unit of U
  const int u = (n + per - 1) / per;
  if (vec) return u <= 1 ? 1 : u <= 2 ? 2 : u <= 3 ? 3 : u <= 4 ? 4 : u <= 6 ? 6 : 8;
  return u <= 1 ? 1 : u <= 2 ? 2 : u <= 4 ? 4 : u <= 8 ? 8 : u <= 16 ? 16 : 32;
}

bool row_vec_ok(const void* a, const void* b, const void* c, int n) {
  return n % 4 == 0 && aligned16(a) && (b == nullptr || aligned16(b)) &&
         (c == nullptr || aligned16(c));
}

// Workgroups (4 waves, one row each) for the softmax and LayerNorm-forward row kernels, at most
// 2^20 of them (the kernels stride over the rest).
dim3 row_grid(int64_t rows) {
  return dim3((unsigned)std::min<int64_t>((rows + 3) / 4, (int64_t)1 << 20));
}

// Workgroups of the long-row kernels (one row each), at most 2^20; they stride over the rest.
dim3 long_row_grid(int64_t rows) {
  return dim3((unsigned)std::min<int64_t>(rows, (int64_t)1 << 20));
}

#define CTA_ROW_SWITCH(KERNEL, VEC, U, GRID, ST, ...)                                        \
  do {                                                                                      \
    if (VEC) {                                                                              \
      switch (U) {                                                                          \
        case 1: hipLaunchKernelGGL((KERNEL<1, true>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 2: hipLaunchKernelGGL((KERNEL<2, true>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 3: hipLaunchKernelGGL((KERNEL<3, true>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 4: hipLaunchKernelGGL((KERNEL<4, true>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 6: hipLaunchKernelGGL((KERNEL<6, true>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        default: hipLaunchKernelGGL((KERNEL<8, true>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
      }                                                                                     \
    } else {                                                                                \
      switch (U) {                                                                          \
        case 1: hipLaunchKernelGGL((KERNEL<1, false>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 2: hipLaunchKernelGGL((KERNEL<2, false>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 4: hipLaunchKernelGGL((KERNEL<4, false>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 8: hipLaunchKernelGGL((KERNEL<8, false>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        case 16: hipLaunchKernelGGL((KERNEL<16, false>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
        default: hipLaunchKernelGGL((KERNEL<32, false>), GRID, dim3(256), 0, ST, __VA_ARGS__); break; \
      }                                                                                     \
    }                                                                                       \
  } while (0)

}  // namespace

// Shared with the naive attention: softmax over contiguous rows (in place allowed).
int zero_floats(float* p, int64_t n, hipStream_t st) {
  if (n <= 0) return CTA_OK;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(grid), dim3(256), 0, st, p, n);
  return check_launch("zero fill");
}

int softmax_rows(const float* x, float* y, int64_t rows, int64_t n, hipStream_t st) {
  if (rows == 0 || n == 0) return CTA_OK;
  if (n > INT32_MAX || rows > ((int64_t)1 << 40)) return fail(CTA_ERR_INVALID_ARGUMENT, "softmax size out of range");
  if (n <= kMaxRegCols) {
    const bool vec = row_vec_ok(x, y, nullptr, (int)n);
    const int u = units_for((int)n, vec);
    CTA_ROW_SWITCH(softmax_fwd_rows, vec, u, row_grid(rows), st, x, y, rows, (int)n);
  } else {
    hipLaunchKernelGGL(softmax_fwd_long, long_row_grid(rows), dim3(256), 0, st, x, y, rows,
                       (int)n);
  }
  return check_launch("softmax");
}

int softmax_bwd_rows_launch(const float* p, const float* dp, float* dx, int64_t rows, int64_t n,
                            hipStream_t st) {
  if (rows == 0 || n == 0) return CTA_OK;
  if (n > INT32_MAX) return fail(CTA_ERR_INVALID_ARGUMENT, "softmax size out of range");
  if (n <= kMaxRegCols) {
    const bool vec = row_vec_ok(p, dp, dx, (int)n);
    const int u = units_for((int)n, vec);
    CTA_ROW_SWITCH(softmax_bwd_rows, vec, u, row_grid(rows), st, p, dp, dx, rows, (int)n);
  } else {
    hipLaunchKernelGGL(softmax_bwd_long, long_row_grid(rows), dim3(256), 0, st, p, dp, dx,
                       rows, (int)n);
  }
  return check_launch("softmax_bwd");
}

// Waves per workgroup of the row-register backward for n columns (see ln_bwd_waves).
int ln_bwd_waves_for(int n, bool vec) {
  const int u = units_for(n, vec);
  return u * (vec ? 4 : 1) <= 12 ? 16 : 8;
}

// Workgroups of the row-register backward: two rows per wave while that needs at most
// kLnBwdMaxBlocks workgroups, more rows per wave beyond.
int64_t ln_bwd_blocks(int64_t rows, int waves) {
  return std::max<int64_t>(1, std::min<int64_t>(kLnBwdMaxBlocks, (rows + 2 * waves - 1) / (2 * waves)));
}

int64_t layernorm_bwd_workspace_floats(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  // the partial rows of either register layout (the launch picks one by alignment)
  const int64_t chunks = n <= kMaxRegCols
                            ? std::max(ln_bwd_blocks(rows, ln_bwd_waves_for((int)n, true)),
                                       ln_bwd_blocks(rows, ln_bwd_waves_for((int)n, false)))
                            : (rows + kLnLongRowsPerBlock - 1) / kLnLongRowsPerBlock;
  return chunks * 2 * n + colsum_partials_scratch_floats(chunks, 2 * n);
}

}  // namespace cta

using namespace cta;

namespace {
template <bool TANH>
int launch_gelu_fwd(const float* x, float* y, int64_t numel, void* stream, const char* name) {
  if (numel < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (numel == 0) return CTA_OK;
  if (!x || !y) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  if (!aligned16(x) || !aligned16(y))
    return fail(CTA_ERR_LAYOUT, std::string(name) + " needs 16-byte aligned buffers");
  const int64_t n4 = numel / 4;
  hipLaunchKernelGGL(TANH ? gelu_tanh_fwd_kernel : gelu_fwd_kernel, dim3(elementwise_grid(n4)),
                     dim3(256), 0,
                     as_stream(stream), x, y, n4, numel);
  return check_launch(name);
}

template <bool TANH>
int launch_gelu_bwd(const float* x, const float* dy, float* dx, int64_t numel, void* stream,
                    const char* name) {
  if (numel < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (numel == 0) return CTA_OK;
  if (!x || !dy || !dx) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  if (!aligned16(x) || !aligned16(dy) || !aligned16(dx))
    return fail(CTA_ERR_LAYOUT, std::string(name) + " needs 16-byte aligned buffers");
  const int64_t n4 = numel / 4;
  hipLaunchKernelGGL(TANH ? gelu_tanh_bwd_kernel : gelu_bwd_kernel, dim3(elementwise_grid(n4)),
                     dim3(256), 0,
                     as_stream(stream), x, dy, dx, n4, numel);
  return check_launch(name);
}
}  // namespace

extern "C" int cta_device_copy(const float* src, float* dst, int64_t n, void* stream) {
  if (n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (n == 0) return CTA_OK;
  if (!src || !dst) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  if (n % 4 != 0 || !aligned16(src) || !aligned16(dst))
    return fail(CTA_ERR_LAYOUT, "device_copy needs n % 4 == 0 and 16-byte aligned buffers");
  hipLaunchKernelGGL(device_copy_kernel, dim3(elementwise_grid(n / 4)), dim3(256), 0,
                     as_stream(stream), src, dst, n / 4);
  return check_launch("device_copy");
}

extern "C" int cta_gelu_fwd(const float* x, float* y, int64_t numel, void* stream) {
  return launch_gelu_fwd<false>(x, y, numel, stream, "gelu_activation");
}

extern "C" int cta_gelu_bwd(const float* x, const float* dy, float* dx, int64_t numel,
                            void* stream) {
  return launch_gelu_bwd<false>(x, dy, dx, numel, stream, "gelu_activation_bwd");
}

extern "C" int cta_gelu_tanh_fwd(const float* x, float* y, int64_t numel, void* stream) {
  return launch_gelu_fwd<true>(x, y, numel, stream, "gelu_tanh_activation");
}

extern "C" int cta_gelu_tanh_bwd(const float* x, const float* dy, float* dx, int64_t numel,
                                 void* stream) {
  return launch_gelu_bwd<true>(x, dy, dx, numel, stream, "gelu_tanh_activation_bwd");
}

extern "C" int cta_softmax_fwd(const float* x, float* y, int64_t rows, int64_t n, void* stream) {
  if (rows < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (rows * n > 0 && (!x || !y)) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  return softmax_rows(x, y, rows, n, as_stream(stream));
}

extern "C" int cta_softmax_bwd(const float* probs, const float* dp, float* dx, int64_t rows,
                               int64_t n, void* stream) {
  if (rows < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (rows * n > 0 && (!probs || !dp || !dx)) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  return softmax_bwd_rows_launch(probs, dp, dx, rows, n, as_stream(stream));
}

namespace {
// LayerNorm forward over rows of x, or of x + f (stored to xsum) when f is given.
int ln_fwd(const float* x, const float* f, const float* gamma, const float* beta, int64_t rows,
           int64_t n, float eps, float* xsum, float* y, float* mean, float* rstd, void* stream) {
  if (rows < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (rows == 0) return CTA_OK;
  if (n == 0) return fail(CTA_ERR_INVALID_ARGUMENT, "layernorm over an empty dimension");
  if (n > INT32_MAX) return fail(CTA_ERR_INVALID_ARGUMENT, "layernorm size out of range");
  if (!x || !gamma || !beta || !y || !mean || !rstd || (f && !xsum))
    return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  hipStream_t st = as_stream(stream);
  if (n <= kMaxRegCols) {
    const bool vec = row_vec_ok(x, y, gamma, (int)n) && aligned16(beta) &&
                     (!f || (aligned16(f) && aligned16(xsum)));
    const int u = units_for((int)n, vec);
    if (f) {
#define CTA_ADD_LN(U_, V_)                                                                     \
  hipLaunchKernelGGL((layernorm_fwd_rows<U_, V_, true>), row_grid(rows), dim3(256), 0, st, x,    \
                     gamma, beta, y, mean, rstd, rows, (int)n, eps, f, xsum)
      if (vec) {
        switch (u) {
          case 1: CTA_ADD_LN(1, true); break;
          case 2: CTA_ADD_LN(2, true); break;
          case 3: CTA_ADD_LN(3, true); break;
          case 4: CTA_ADD_LN(4, true); break;
          case 6: CTA_ADD_LN(6, true); break;
          default: CTA_ADD_LN(8, true); break;
        }
      } else {
        switch (u) {
          case 1: CTA_ADD_LN(1, false); break;
          case 2: CTA_ADD_LN(2, false); break;
          case 4: CTA_ADD_LN(4, false); break;
          case 8: CTA_ADD_LN(8, false); break;
          case 16: CTA_ADD_LN(16, false); break;
          default: CTA_ADD_LN(32, false); break;
        }
      }
#undef CTA_ADD_LN
    } else {
      CTA_ROW_SWITCH(layernorm_fwd_rows, vec, u, row_grid(rows), st, x, gamma, beta, y, mean,
                     rstd, rows, (int)n, eps);
    }
  } else {
    hipLaunchKernelGGL(layernorm_fwd_long, long_row_grid(rows), dim3(256), 0, st, x, gamma,
                       beta, y, mean, rstd, rows, (int)n, eps, f, xsum);
  }
  return check_launch("layernorm_fwd");
}
}  // namespace

extern "C" int cta_layernorm_fwd(const float* x, const float* gamma, const float* beta,
                                 int64_t rows, int64_t n, float eps, float* y, float* mean,
                                 float* rstd, void* stream) {
  return ln_fwd(x, nullptr, gamma, beta, rows, n, eps, nullptr, y, mean, rstd, stream);
}

extern "C" int cta_add_layernorm_fwd(const float* x, const float* f, const float* gamma,
                                     const float* beta, int64_t rows, int64_t n, float eps,
                                     float* xsum, float* y, float* mean, float* rstd,
                                     void* stream) {
  if (rows > 0 && n > 0 && !f) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  return ln_fwd(x, f, gamma, beta, rows, n, eps, xsum, y, mean, rstd, stream);
}

extern "C" int64_t cta_layernorm_bwd_workspace(int64_t rows, int64_t n) {
  return layernorm_bwd_workspace_floats(rows, n) * (int64_t)sizeof(float);
}

namespace {
// LayerNorm backward; with dres, dx also receives dres (the residual path's gradient).
int ln_bwd(const float* x, const float* gamma, const float* mean, const float* rstd,
           const float* dy, const float* dres, int64_t rows, int64_t n, float* dx, float* dgamma,
           float* dbeta, float* workspace, void* stream) {
  if (rows < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (n == 0) return CTA_OK;
  if (n > INT32_MAX) return fail(CTA_ERR_INVALID_ARGUMENT, "layernorm size out of range");
  if (!dgamma || !dbeta) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  hipStream_t st = as_stream(stream);
  if (rows == 0) {
    if (int rc = zero_floats(dgamma, n, st)) return rc;
    return zero_floats(dbeta, n, st);
  }
  if (!x || !gamma || !mean || !rstd || !dy || !dx || !workspace)
    return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  if (n <= kMaxRegCols) {
    const bool vec = row_vec_ok(x, dy, dx, (int)n) && aligned16(gamma) && (!dres || aligned16(dres));
    const int u = units_for((int)n, vec);
    const int waves = ln_bwd_waves_for((int)n, vec);
    const int64_t blocks = ln_bwd_blocks(rows, waves);
    const int rows_per_wave = (int)((rows + blocks * waves - 1) / (blocks * waves));
#define CTA_LN_BWD(U_, V_)                                                                     \
  do {                                                                                         \
    if (dres)                                                                                  \
      hipLaunchKernelGGL((layernorm_bwd_rows<U_, V_, true>), dim3((unsigned)blocks),           \
                         dim3(64 * ln_bwd_waves<U_, V_>()), 0, st, x, gamma, mean, rstd, dy,   \
                         dx, workspace, rows, (int)n, rows_per_wave, dres);                    \
    else                                                                                       \
      hipLaunchKernelGGL((layernorm_bwd_rows<U_, V_>), dim3((unsigned)blocks),                 \
                         dim3(64 * ln_bwd_waves<U_, V_>()), 0, st, x, gamma, mean, rstd, dy,   \
                         dx, workspace, rows, (int)n, rows_per_wave);                          \
  } while (0)
    if (vec) {
      switch (u) {
        case 1: CTA_LN_BWD(1, true); break;
        case 2: CTA_LN_BWD(2, true); break;
        case 3: CTA_LN_BWD(3, true); break;
        case 4: CTA_LN_BWD(4, true); break;
        case 6: CTA_LN_BWD(6, true); break;
        default: CTA_LN_BWD(8, true); break;
      }
    } else {
      switch (u) {
        case 1: CTA_LN_BWD(1, false); break;
        case 2: CTA_LN_BWD(2, false); break;
        case 4: CTA_LN_BWD(4, false); break;
        case 8: CTA_LN_BWD(8, false); break;
        case 16: CTA_LN_BWD(16, false); break;
        default: CTA_LN_BWD(32, false); break;
      }
    }
#undef CTA_LN_BWD
    if (int rc = check_launch("layernorm_bwd")) return rc;
    return colsum_partials_launch(workspace, blocks, 2 * n, dgamma, dbeta, n, st,
                                  workspace + blocks * 2 * n);
  } else {
    hipLaunchKernelGGL(layernorm_bwd_long, long_row_grid(rows), dim3(256), 0, st, x, gamma,
                       mean, rstd, dy, dx, rows, (int)n, dres);
    const int64_t chunks = (rows + kLnLongRowsPerBlock - 1) / kLnLongRowsPerBlock;
    if (chunks > 65535) return fail(CTA_ERR_INVALID_ARGUMENT, "too many rows for layernorm_bwd");
    hipLaunchKernelGGL(layernorm_colpart_long, dim3((unsigned)((n + 255) / 256), (unsigned)chunks),
                       dim3(256), 0, st, x, mean, rstd, dy, workspace, rows, (int)n,
                       kLnLongRowsPerBlock);
    if (int rc = check_launch("layernorm_bwd")) return rc;
    return colsum_partials_launch(workspace, chunks, 2 * n, dgamma, dbeta, n, st,
                                  workspace + chunks * 2 * n);
  }
  return check_launch("layernorm_bwd");
}
}  // namespace

extern "C" int cta_layernorm_bwd(const float* x, const float* gamma, const float* mean,
                                 const float* rstd, const float* dy, int64_t rows, int64_t n,
                                 float* dx, float* dgamma, float* dbeta, float* workspace,
                                 void* stream) {
  return ln_bwd(x, gamma, mean, rstd, dy, nullptr, rows, n, dx, dgamma, dbeta, workspace, stream);
}

extern "C" int cta_add_layernorm_bwd(const float* xsum, const float* gamma, const float* mean,
                                     const float* rstd, const float* dy, const float* dres,
                                     int64_t rows, int64_t n, float* dx, float* dgamma,
                                     float* dbeta, float* workspace, void* stream) {
  if (rows > 0 && n > 0 && !dres) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  return ln_bwd(xsum, gamma, mean, rstd, dy, dres, rows, n, dx, dgamma, dbeta, workspace, stream);
}
