// FlashAttention-2 forward, FP32, CDNA4 MFMA.
//
// Semantics follow Transformer_kernels/flash_attention.cuh:27-170 (online softmax over
// K/V tiles; O = sum_j e^{S_ij - m_i} v_j / l_i and L_i = m_i + ln l_i with S = q.k/sqrt(hs),
// causal mask j > i, rows beyond T never written).  The algorithm is re-designed for
// gfx950:
//
//  * A workgroup owns BM = 128 query rows (4 waves x 32 rows; 64 rows of 2 waves for short
//    causal heads).  K/V tiles of BN rows are
//    staged global -> registers -> LDS, double buffered, one barrier per tile.
//  * Each wave computes S^T = K Q^T with v_mfma_f32_32x32x2_f32.  In the MFMA output layout
//    lane l then holds 16 scores of query row (l % 32) — one row per lane — so the row max
//    needs one in-lane max over 16 registers and one exchange with the other wave half.
//  * O^T = V^T P^T reuses the score registers directly as the B operand: the K index of the
//    second MFMA is permuted to match the output layout of the first, and V is read from LDS
//    in the same permuted order.  P never leaves registers.
//  * Exponentials use exp2 with log2(e) folded into the scale; L is exported in natural log.
//  * Lazy rescaling: the running max m used as the exponent offset only moves when some row
//    of the wave sees a tile max more than 2^8 above it (a wave-uniform vote).  Otherwise the
//    tile is exponentiated against the stale m, so every p <= 2^8 and the O accumulator and
//    row sum stay exact multiples of the same e^{-m}; O = acc / l and L = m + ln l are
//    unchanged.  This removes the per-tile rescale of the O registers from the common path.
//  * The max / sum across the two wave halves use v_permlane32_swap (no LDS round trip).
//  * Workgroup ids are remapped so each XCD walks a contiguous run of a head-major work list:
//    the workgroups resident on one XCD share a few heads' K/V in its L2.  With a causal mask a
//    workgroup takes the query-tile pair (n-1-p, p), so all workgroups cost the same and the
//    head-major order leaves no long tiles for the end; on grids too small for the pairs to
//    fill the resident slots each XCD instead takes single tiles of its heads longest first
//    (lpt_heads).
#include "cta_common.hpp"

namespace cta {
namespace {

struct RowStrides {
  int64_t b, h, t;  // element strides of the batch, head and time axes (d-stride is 1)
};

template <int HS>
struct FwdTile;
template <> struct FwdTile<32> { static constexpr int BN = 32; static constexpr int MINW = 2; };
template <> struct FwdTile<64> { static constexpr int BN = 32; static constexpr int MINW = 2; };
template <> struct FwdTile<128> { static constexpr int BN = 32; static constexpr int MINW = 1; };

// NSPLIT > 1: each work item (query-tile pair, or tile) is run by NSPLIT workgroups, parts 0 ..
// NSPLIT - 1, each over a contiguous share of the item's K/V stages (in the item's stage order,
// across its passes).  Each writes its share's normalised O and L = m + ln l (O = 0, L = -inf
// where it saw no key): part 0 into O / L, part k densely into the (k - 1)th slabs of Os / Ls;
// fa2_fwd_merge_kernel then combines them.
template <int HS, bool CAUSAL, int WAVES = 4, int NSPLIT = 1>
__global__ __launch_bounds__(64 * WAVES, FwdTile<HS>::MINW) void fa2_fwd_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ L, int nh, int T, int BH, int n_qtiles,
    RowStrides sq, RowStrides sk, RowStrides sv, RowStrides so, float scale, float scale_log2,
    float rescale_gap, float* __restrict__ Os = nullptr, float* __restrict__ Ls = nullptr,
    int heads_per_xcd = 0) {
  constexpr int BN = FwdTile<HS>::BN;
  constexpr int THREADS = 64 * WAVES;
  constexpr int BM = 32 * WAVES;  // query rows per workgroup, 32 per wave
  constexpr int H2 = HS / 2;    // d values per lane half
  constexpr int KP = HS + 4;    // LDS pitch (floats) of a K row: conflict-free 16-byte row reads
  constexpr int VP = HS + 8;    // LDS pitch of a V row: the two wave halves read rows 4 apart
  constexpr int KTILE = BN * KP;
  constexpr int VTILE = BN * VP;
  constexpr int F4_ROW = HS / 4;
  constexpr int LOADS = BN * F4_ROW / THREADS;
  static_assert(BN * F4_ROW % THREADS == 0, "tile must split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) float smem[2 * (KTILE + VTILE)];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  // Work items are head-major and spread over XCDs.  Causal: one item = the query-tile pair
  // (n-1-p, p), so every item costs n+1 tile units and the dynamic dispatch has no tail.
  // Causal with heads_per_xcd > 0 (unsplit): one item = one query tile, longest first per XCD
  // (lpt_tile; grid BH * n_qtiles).
  constexpr bool SPLIT = NSPLIT > 1;
  int bh, part = 0;
  int qa, qb = -1;  // the item's query tiles, in pass order (qb < 0: one pass)
  if (CAUSAL && !SPLIT && heads_per_xcd > 0) {
    int rank;
    lpt_tile(blockIdx.x, heads_per_xcd, bh, rank);
    qa = n_qtiles - 1 - rank;
  } else {
    const int per_head = CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles;
    const int n_items = BH * per_head * NSPLIT;
    const int w = xcd_work_item(blockIdx.x, n_items);
    if (w >= n_items) return;
    const int item = SPLIT ? w / NSPLIT : w;
    part = SPLIT ? w - item * NSPLIT : 0;  // an item's parts are neighbours: one XCD
    bh = item / per_head;
    const int p = item - bh * per_head;
    qa = CAUSAL ? n_qtiles - 1 - p : p;
    if (CAUSAL && n_qtiles - 1 - p != p) qb = p;
  }
  const int b = bh / nh, h = bh - b * nh;

  const float* Qb = Q + b * sq.b + h * sq.h;
  const float* Kb = K + b * sk.b + h * sk.h;
  const float* Vb = V + b * sv.b + h * sv.h;

  const int n_pass = qb >= 0 ? 2 : 1;
  auto qt_of = [&](int pass) { return pass == 0 ? qa : qb; };
  auto stages_of = [&](int qt) {
    return ((CAUSAL ? min(T, (qt + 1) * BM) : T) + BN - 1) / BN;
  };
  // SPLIT: this part's positions [g0, g1) in the item's list of stages (pass 0's, then pass
  // 1's): boundaries at ceil(total k / NSPLIT).
  int g0 = 0, g1 = 0, pos = 0;
  if constexpr (SPLIT) {
    int total = 0;
    for (int pass = 0; pass < n_pass; ++pass) total += stages_of(qt_of(pass));
    g0 = (total * part + NSPLIT - 1) / NSPLIT;
    g1 = (total * (part + 1) + NSPLIT - 1) / NSPLIT;
  }
  for (int pass = 0; pass < n_pass; ++pass) {
  const int qt = qt_of(pass);
  const int i0 = qt * BM + wave * 32;  // first query row of this wave
  const int my_i = i0 + col;           // query row owned by this lane

  float qf[H2];
  if (my_i < T) {
    const float* qp = Qb + (int64_t)my_i * sq.t + half * H2;
#pragma unroll
    for (int c = 0; c < H2 / 4; ++c) {
      float4 x = ld4(qp + 4 * c);
      qf[4 * c + 0] = x.x; qf[4 * c + 1] = x.y; qf[4 * c + 2] = x.z; qf[4 * c + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < H2; ++c) qf[c] = 0.0f;
  }

  f32x16 oacc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) oacc[d] = zero16();
  float m_run = -INFINITY;  // exponent offset of row my_i (raw q.k units), lazily updated
  float l_run = 0.0f;       // this lane's partial row sum (its half of the columns)
  // The exponents are (S - m) s log2(e): the subtraction comes first, so the row maximum gets
  // exactly 2^0 at any score magnitude, as the reference's expf(S - m) does
  // (flash_attention.cuh:130-134).  Folding m into one rounded offset, fma(S, c, -m c), cost the
  // same but let the offset's rounding error (growing with |m|) overflow rows past |m| ~ 2^20.

  const int n_stages = stages_of(qt);
  // the stages [i_begin, i_end) of this pass that this part runs (all of them unless SPLIT)
  const int i_begin = SPLIT ? min(max(g0 - pos, 0), n_stages) : 0;
  const int i_end = SPLIT ? min(max(g1 - pos, 0), n_stages) : n_stages;
  pos += n_stages;

  float4 kst[LOADS], vst[LOADS];
  // K/V rows of a stage through buffer resources over its valid rows (scalar base and extent;
  // the lanes' offsets are the same every stage): rows past T read as zero.
  auto gload = [&](int stage) {
    const int j0 = stage * BN;
    const int rows = min(BN, T - j0);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(Kb + (int64_t)j0 * sk.t, rows, sk.t, HS);
    const __amdgpu_buffer_rsrc_t rv = rows_rsrc(Vb + (int64_t)j0 * sv.t, rows, sv.t, HS);
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + THREADS * u;
      const int r = f / F4_ROW, c4 = f % F4_ROW;
      kst[u] = ld4_buffer(rk, (r * (int)sk.t + 4 * c4) * 4);
      vst[u] = ld4_buffer(rv, (r * (int)sv.t + 4 * c4) * 4);
    }
  };
  auto lstore = [&](int buf) {
    float* ks = smem + buf * (KTILE + VTILE);
    float* vs = ks + KTILE;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + THREADS * u;
      const int r = f / F4_ROW, c4 = f % F4_ROW;
      st4(ks + r * KP + 4 * c4, kst[u]);
      st4(vs + r * VP + 4 * c4, vst[u]);
    }
  };

  // Stage order.  With a causal mask the second (short) pass walks the K/V stages downward
  // from its last: every workgroup of a head in its first pass reads stage t at step t, and
  // every one in its second pass reads stage 4n+3-t (n query tiles; t counted from the item's
  // start), so the workgroups of a head share each K/V stage in L2.  The direction belongs to
  // the tile (the short one of its pair walks down), so longest-first single tiles sum in the
  // same order as pairs and give the same bits.
  const bool down = CAUSAL && qt < n_qtiles - 1 - qt;
  auto stage_at = [&](int i) { return down ? n_stages - 1 - i : i; };
  if (i_begin < i_end) {  // workgroup-uniform
    gload(stage_at(i_begin));
    lstore(0);
  }
  __syncthreads();

  for (int i = i_begin; i < i_end; ++i) {
    const int s = stage_at(i);
    const int buf = (i - i_begin) & 1;
    if (i + 1 < i_end) gload(stage_at(i + 1));
    const float* ks = smem + buf * (KTILE + VTILE);
    const float* vs = ks + KTILE;

#pragma unroll
    for (int sub = 0; sub < BN / 32; ++sub) {
      const int jj0 = s * BN + sub * 32;
      if (jj0 >= T) continue;                      // ragged tail: nothing left in this stage
      if (CAUSAL && jj0 > i0 + 31) continue;       // tile entirely above this wave's diagonal

      // S^T tile: sacc[r] = q_{my_i} . k_{jj0 + R(r, half)}
      f32x16 sacc = zero16();
      const float* krow = ks + (sub * 32 + col) * KP + half * H2;
#pragma unroll
      for (int c = 0; c < H2 / 4; ++c) {
        const float4 kv = ld4(krow + 4 * c);
        sacc = mfma32(kv.x, qf[4 * c + 0], sacc);
        sacc = mfma32(kv.y, qf[4 * c + 1], sacc);
        sacc = mfma32(kv.z, qf[4 * c + 2], sacc);
        sacc = mfma32(kv.w, qf[4 * c + 3], sacc);
      }

      const bool need_mask = (CAUSAL && jj0 + 31 > i0) || (jj0 + 32 > T);
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = jj0 + mfma_row(r, half);
          if ((CAUSAL && j > my_i) || j >= T) sacc[r] = -INFINITY;
        }
      }

      float mt = sacc[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mt = fmaxf(mt, sacc[r]);
      mt = max_halves(mt);
      // rescale_gap = 8 / scale_log2: a tile max within 2^8 of m keeps the old offset.
      // The first tile always rescales (m_run = -inf), with alpha = 0 on zero accumulators.
      if (__any(mt > m_run + rescale_gap)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = fast_exp2((m_run - m_new) * scale_log2);
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < HS / 32; ++d) oacc[d] *= alpha;
        m_run = m_new;
      }
      float psum = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2((sacc[r] - m_run) * scale_log2);
        sacc[r] = p;
        psum += p;
      }
      l_run += psum;

#pragma unroll
      for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
          const float a = vs[(sub * 32 + mfma_row(kk, half)) * VP + d * 32 + col];
          oacc[d] = mfma32(a, sacc[kk], oacc[d]);
        }
      }
    }

    if (i + 1 < i_end) lstore(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = sum_halves(l_run);
  if (my_i < T) {
    if constexpr (SPLIT) {
      // A part may have seen no key of this row (l = 0): O = 0, L = -inf, which the merge
      // weighs by e^{-inf} = 0.
      const bool seen = l_tot > 0.0f;
      const float inv = seen ? 1.0f / l_tot : 0.0f;
      const int64_t slab = (int64_t)(part - 1) * BH * T;  // part k >= 1: slab k - 1
      float* op = part ? Os + (slab + (int64_t)bh * T + my_i) * HS
                       : O + b * so.b + h * so.h + (int64_t)my_i * so.t;
#pragma unroll
      for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int dc = d * 32 + 8 * g + 4 * half;
          st4(op + dc, make_float4(oacc[d][4 * g + 0] * inv, oacc[d][4 * g + 1] * inv,
                                   oacc[d][4 * g + 2] * inv, oacc[d][4 * g + 3] * inv));
        }
      }
      if (half == 0)
        (part ? Ls + slab : L)[(int64_t)bh * T + my_i] =
            seen ? m_run * scale + logf(l_tot) : -INFINITY;
    } else {
      float* op = O + b * so.b + h * so.h + (int64_t)my_i * so.t;
#pragma unroll
      for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int dc = d * 32 + 8 * g + 4 * half;
          st4(op + dc, make_float4(oacc[d][4 * g + 0] / l_tot, oacc[d][4 * g + 1] / l_tot,
                                   oacc[d][4 * g + 2] / l_tot, oacc[d][4 * g + 3] / l_tot));
        }
      }
      if (half == 0) L[(int64_t)bh * T + my_i] = m_run * scale + logf(l_tot);
    }
  }
  }  // pass: the K/V loop ended on a barrier, so the next pass may refill LDS
}

// Merge of the NSPLIT parts of a split forward, row by row in a fixed order (part 0, 1, ...):
// L = ln(sum_k e^{Lk}), taken about their maximum, and O = sum_k e^{Lk - L} Ok; part 0 in
// O / L (O through its strides), part k >= 1 dense in slab k - 1 of Os / Ls.  HS / 4 lanes per
// row, one float4 each.
template <int HS, int NSPLIT>
__global__ __launch_bounds__(256) void fa2_fwd_merge_kernel(float* __restrict__ O,
                                                            float* __restrict__ L,
                                                            const float* __restrict__ Os,
                                                            const float* __restrict__ Ls, int nh,
                                                            int T, int64_t rows, RowStrides so) {
  constexpr int G = HS / 4;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / G;
  if (row >= rows) return;
  const int c4 = (int)(gid % G);
  const int64_t bh = row / T;
  const int t = (int)(row - bh * T);
  const int64_t b = bh / nh, h = bh - b * nh;
  float lk[NSPLIT];
  lk[0] = L[row];
#pragma unroll
  for (int k = 1; k < NSPLIT; ++k) lk[k] = Ls[(int64_t)(k - 1) * rows + row];
  float m = lk[0];  // finite: every row sees key 0 in one of the parts
#pragma unroll
  for (int k = 1; k < NSPLIT; ++k) m = fmaxf(m, lk[k]);
  float e[NSPLIT], sum = 0.0f;
#pragma unroll
  for (int k = 0; k < NSPLIT; ++k) {
    e[k] = expf(lk[k] - m);
    sum += e[k];
  }
  const float inv = 1.0f / sum;
  float* op = O + b * so.b + h * so.h + (int64_t)t * so.t + 4 * c4;
  // acc = w_{N-1} O_{N-1}, then fma in the weights of parts N-2 .. 0
  const float wl = e[NSPLIT - 1] * inv;
  const float4 cl = ld4(Os + ((int64_t)(NSPLIT - 2) * rows + row) * HS + 4 * c4);
  float4 acc = make_float4(wl * cl.x, wl * cl.y, wl * cl.z, wl * cl.w);
#pragma unroll
  for (int k = NSPLIT - 2; k >= 1; --k) {
    const float wk = e[k] * inv;
    const float4 c = ld4(Os + ((int64_t)(k - 1) * rows + row) * HS + 4 * c4);
    acc = make_float4(fmaf(wk, c.x, acc.x), fmaf(wk, c.y, acc.y), fmaf(wk, c.z, acc.z),
                      fmaf(wk, c.w, acc.w));
  }
  const float w0 = e[0] * inv;
  const float4 a = ld4(op);
  st4(op, make_float4(fmaf(w0, a.x, acc.x), fmaf(w0, a.y, acc.y), fmaf(w0, a.z, acc.z),
                      fmaf(w0, a.w, acc.w)));
  if (c4 == 0) L[row] = m + logf(sum);
}

// The forward splits each work item's K/V stages over NSPLIT workgroups when its grid would hold
// fewer than two waves per SIMD (1024 SIMDs): enough parts to fill the waves per SIMD its
// registers and LDS allow (three at hs 32 / 64, two at hs 128), each part keeping at least
// kSplitMinStages stages; the merge pass is the cost.  A/B in one process against the unsplit
// forward: B4 H4 N4096 causal 0.3306 -> 0.3042 ms with two parts (+8.7%), B2 H4 N4096
// non-causal +7.3%; at T = 256 (B64 H6, 8 stages per row) two parts were 30% slower, the merge
// outweighing the work, hence the minimum.
constexpr int kSimds = 1024;
constexpr int kSplitMinStages = 16;

template <int HS, bool CAUSAL>
int fwd_waves(int T) {
  return (HS == 64 && CAUSAL && T <= 512) ? 2 : 4;
}

// Parts per work item: 1 (no split), 2 or 3.
template <int HS, bool CAUSAL>
int fwd_nsplit(int T, int BH) {
  const int waves = fwd_waves<HS, CAUSAL>(T);
  const int n_qtiles = (T + 32 * waves - 1) / (32 * waves);
  const int64_t w = (int64_t)(CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles) * BH * waves;
  if (w >= 2 * kSimds) return 1;
  const int occ = HS == 128 ? 2 : 3;  // waves per SIMD the unsplit kernel can hold
  int n = (int)std::min<int64_t>(occ, (occ * kSimds + w - 1) / w);
  n = std::min(n, T / FwdTile<HS>::BN / kSplitMinStages);
  return n >= 2 ? n : 1;
}

// Longest-first tiles (lpt_heads), A/B in one process against pairs (bitwise-equal outputs):
// B64 H6 T256 causal +9%, B16 H8 T512 +29% (two-wave workgroups, every tile resident at once).
// The split forward, where it applies, beats both (B2 H8 N1024: 0.060 ms split, 0.084 ms
// longest-first), so a split launch keeps the pairs.

template <int HS, bool CAUSAL>
void launch_fwd(const float* q, const float* k, const float* v, float* o, float* l, int nh,
                int T, int BH, RowStrides sq, RowStrides sk, RowStrides sv, RowStrides so,
                float scale, hipStream_t stream, float* split_ws = nullptr) {
  auto run = [&]<int WAVES>() {
    const int n_qtiles = (T + 32 * WAVES - 1) / (32 * WAVES);
    const int64_t items = (int64_t)(CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles) * BH;
    const int nsplit = split_ws != nullptr ? fwd_nsplit<HS, CAUSAL>(T, BH) : 1;
    auto split = [&]<int NS>() {
      const int64_t rows = (int64_t)BH * T;
      float* Os = split_ws;
      float* Ls = split_ws + (NS - 1) * rows * HS;
      hipLaunchKernelGGL((fa2_fwd_kernel<HS, CAUSAL, WAVES, NS>), dim3(xcd_grid(NS * items)),
                         dim3(64 * WAVES), 0, stream, q, k, v, o, l, nh, T, BH, n_qtiles, sq, sk,
                         sv, so, scale, scale * kLog2e, 8.0f / (scale * kLog2e), Os, Ls);
      hipLaunchKernelGGL((fa2_fwd_merge_kernel<HS, NS>),
                         dim3((unsigned)((rows * (HS / 4) + 255) / 256)), dim3(256), 0, stream, o,
                         l, Os, Ls, nh, T, rows, so);
    };
    if (nsplit == 3) {
      split.template operator()<3>();
      return;
    }
    if (nsplit == 2) {
      split.template operator()<2>();
      return;
    }
    // Slots counted at three waves per SIMD for hs 32 / 64 (the four-wave kernel's 160 VGPRs
    // hold three; the two-wave one's 186 hold two, but measured, its longest-first tiles win at
    // B64 H6 T256, 1.5 rounds of them at two waves, +9%, and lose at B8 H32 T512, 2 rounds, -3%,
    // which the three-wave count separates).
    const int lpt = CAUSAL ? lpt_heads(BH, n_qtiles, WAVES, HS == 128 ? 1 : 3) : 0;
    hipLaunchKernelGGL((fa2_fwd_kernel<HS, CAUSAL, WAVES>),
                       dim3(lpt > 0 ? (unsigned)(BH * n_qtiles) : xcd_grid(items)),
                       dim3(64 * WAVES), 0, stream, q, k, v, o, l, nh, T, BH, n_qtiles, sq, sk,
                       sv, so, scale, scale * kLog2e, 8.0f / (scale * kLog2e), nullptr, nullptr,
                       lpt);
  };
  // Short causal heads (hs 64, T <= 512) run two waves (64 query rows) per workgroup: fewer
  // waves idle at each K/V stage's barrier along the diagonal, and the query-tile pairs balance
  // over twice as many workgroups.  A/B in one process, bitwise-equal outputs: +13% at T = 256,
  // +7% at 512, within 1.5% either way at 1024 and 2048.
  if constexpr (HS == 64 && CAUSAL) {
    if (T <= 512) {
      run.template operator()<2>();
      return;
    }
  }
  run.template operator()<4>();
}

}  // namespace

// The kernels read 16-byte row segments (unit d-stride, strides divisible by 4, 16-byte aligned
// base) and address a stage of up to 64 rows with 32-bit byte offsets (time stride 0 to 2^23).
bool attn_layout_ok(const float* p, const int64_t* s) {
  return p != nullptr && s != nullptr && aligned16(p) && s[3] == 1 && s[0] % 4 == 0 &&
         s[1] % 4 == 0 && s[2] % 4 == 0 && s[2] >= 0 && s[2] < kMaxAttnTimeStride;
}

int check_attn_sizes(int64_t B, int64_t nh, int64_t T, int64_t hs) {
  if (B < 0 || nh < 0 || T < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (hs != 32 && hs != 64 && hs != 128)
    return fail(CTA_ERR_UNSUPPORTED_HEAD_DIM,
                "Unsupported head dimension! Only hs=32, hs=64, and hs=128 are supported.");
  if (B * nh > (int64_t)1 << 24 || T > (int64_t)1 << 24)
    return fail(CTA_ERR_INVALID_ARGUMENT, "size too large");
  return CTA_OK;
}

}  // namespace cta

using namespace cta;

namespace {
template <typename F>
void dispatch_fwd(int64_t hs, int causal, F&& f) {
  if (hs == 32) {
    if (causal) f.template operator()<32, true>();
    else f.template operator()<32, false>();
  } else if (hs == 64) {
    if (causal) f.template operator()<64, true>();
    else f.template operator()<64, false>();
  } else {
    if (causal) f.template operator()<128, true>();
    else f.template operator()<128, false>();
  }
}
}  // namespace

extern "C" int64_t cta_flash_attention_fwd_workspace(int64_t B, int64_t nh, int64_t T,
                                                     int64_t hs, int causal) {
  if (B <= 0 || nh <= 0 || T <= 0 || (hs != 32 && hs != 64 && hs != 128) ||
      B * nh > ((int64_t)1 << 24) || T > ((int64_t)1 << 24))
    return 0;
  int nsplit = 1;
  dispatch_fwd(hs, causal, [&]<int HS, bool C>() { nsplit = fwd_nsplit<HS, C>((int)T, (int)(B * nh)); });
  return (nsplit - 1) * B * nh * T * (hs + 1) * (int64_t)sizeof(float);
}

extern "C" int cta_flash_attention_fwd_ex(const float* q, const int64_t* q_strides,
                                          const float* k, const int64_t* k_strides,
                                          const float* v, const int64_t* v_strides, int64_t B,
                                          int64_t nh, int64_t T, int64_t hs, int causal,
                                          float* o, const int64_t* o_strides, float* l,
                                          void* workspace, int64_t workspace_bytes,
                                          void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (!o || !l) return fail(CTA_ERR_INVALID_ARGUMENT, "null output pointer");
  if (!attn_layout_ok(q, q_strides) || !attn_layout_ok(k, k_strides) ||
      !attn_layout_ok(v, v_strides) || !attn_layout_ok(o, o_strides))
    return fail(CTA_ERR_LAYOUT,
                "flash_attention_fwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                "aligned Q/K/V/O");
  const int64_t need = cta_flash_attention_fwd_workspace(B, nh, T, hs, causal);
  float* split_ws = nullptr;
  if (need > 0 && workspace != nullptr && workspace_bytes >= need) {
    if (!aligned16(workspace))
      return fail(CTA_ERR_LAYOUT, "the workspace must be a 16-byte aligned pointer");
    split_ws = static_cast<float*>(workspace);
  }
  const RowStrides sq{q_strides[0], q_strides[1], q_strides[2]};
  const RowStrides sk{k_strides[0], k_strides[1], k_strides[2]};
  const RowStrides sv{v_strides[0], v_strides[1], v_strides[2]};
  const RowStrides so{o_strides[0], o_strides[1], o_strides[2]};
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  hipStream_t st = as_stream(stream);
  dispatch_fwd(hs, causal, [&]<int HS, bool C>() {
    launch_fwd<HS, C>(q, k, v, o, l, (int)nh, (int)T, (int)(B * nh), sq, sk, sv, so, scale, st,
                      split_ws);
  });
  return check_launch("flash_attention_fwd");
}

extern "C" int cta_flash_attention_fwd_strided(const float* q, const int64_t* q_strides,
                                               const float* k, const int64_t* k_strides,
                                               const float* v, const int64_t* v_strides,
                                               int64_t B, int64_t nh, int64_t T, int64_t hs,
                                               int causal, float* o, const int64_t* o_strides,
                                               float* l, void* stream) {
  return cta_flash_attention_fwd_ex(q, q_strides, k, k_strides, v, v_strides, B, nh, T, hs,
                                    causal, o, o_strides, l, nullptr, 0, stream);
}

extern "C" int cta_flash_attention_fwd(const float* q, const int64_t* q_strides, const float* k,
                                       const int64_t* k_strides, const float* v,
                                       const int64_t* v_strides, int64_t B, int64_t nh,
                                       int64_t T, int64_t hs, int causal, float* o, float* l,
                                       void* stream) {
  const int64_t os[4] = {nh * T * hs, T * hs, hs, 1};  // dense (B, nh, T, hs)
  return cta_flash_attention_fwd_strided(q, q_strides, k, k_strides, v, v_strides, B, nh, T, hs,
                                         causal, o, os, l, stream);
}
