// FlashAttention-2 backward, FP32, CDNA4 MFMA: three atomics-free stages.
//
// Semantics follow Transformer_kernels/flash_attention.cuh:175-504:
//   delta_i = sum_d O_id dO_id                                   (:175-213)
//   P_ij = e^{S_ij - L_i},  dP_ij = dO_i . v_j,  dS_ij = P_ij (dP_ij - delta_i)
//   dQ_i = s * sum_j dS_ij k_j                                   (:216-354)
//   dV_j = sum_i P_ij dO_i,  dK_j = s * sum_i dS_ij q_i          (:357-504)
// with S = s q.k, s = 1/sqrt(hs), and the causal mask j > i.  Each output row is owned by
// exactly one lane, so there are no atomics and results are deterministic.
//
// gfx950 design (same MFMA layout trick as the forward kernel):
//  * dQ stage: a wave owns 32 query rows and keeps q, dO, L and delta of its rows in
//    registers.  It computes S^T = K Q^T and dP^T = V dO^T (one query row per lane), forms
//    dS^T in registers and feeds it straight into dQ^T += K^T dS^T.
//  * dK/dV stage: a wave owns 32 key rows and keeps k and v in registers.  It computes
//    S = Q K^T and dP = dO V^T (one key row per lane) and feeds P and dS straight into
//    dV^T += dO^T P and dK^T += Q^T dS.  Unlike the reference, causal tiles above the
//    diagonal are skipped here too (the reference computes kvEnd but never uses it).
//  * Tiles of the streamed operand (K,V for dQ; Q,dO,L,delta for dK/dV) go
//    global -> registers -> LDS, double buffered, one barrier per tile.
//
// Stored-dS schedule (cta_flash_attention_bwd given a workspace): the reference's dQ stage
// recomputes S and dP, so the three stages run seven tile GEMMs.  With HBM to spare, the
// dK/dV kernel also writes every 32x32 dS tile it forms to a workspace, transposed through
// LDS into the order the dQ kernel reads, and a lean dQ kernel computes dQ = s * dS K from
// it: five GEMMs, still without atomics and bitwise deterministic.  The workspace holds
// whole heads (the lower-triangular tiles only when causal); heads are processed in chunks
// when the caller's workspace cannot hold them all.
#include "cta_common.hpp"

namespace cta {
namespace {

struct RowStrides {
  int64_t b, h, t;
};
struct LStrides {
  int64_t b, h, t;
};

// ------------------------------------------------------------------------------------
// Stage 1: delta.  G = hs/4 lanes share one row (one float4 each).
template <int HS>
__global__ __launch_bounds__(256) void fa2_bwd_delta_kernel(const float* __restrict__ O,
                                                            const float* __restrict__ dO,
                                                            float* __restrict__ delta, int nh,
                                                            int T, int64_t rows, RowStrides so,
                                                            RowStrides sdo) {
  constexpr int G = HS / 4;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / G;
  const int c4 = (int)(gid % G);
  float acc = 0.0f;
  if (row < rows) {
    const int64_t bh = row / T;
    const int t = (int)(row - bh * T);
    const int64_t b = bh / nh, h = bh - b * nh;
    const float4 o = ld4(O + b * so.b + h * so.h + (int64_t)t * so.t + 4 * c4);
    const float4 g = ld4(dO + b * sdo.b + h * sdo.h + (int64_t)t * sdo.t + 4 * c4);
    acc = o.x * g.x + o.y * g.y + o.z * g.z + o.w * g.w;
  }
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (row < rows && c4 == 0) delta[row] = acc;
}

template <int HS>
struct BwdTile;
template <> struct BwdTile<32> { static constexpr int BN = 64; static constexpr int MINW = 2; };
template <> struct BwdTile<64> { static constexpr int BN = 64; static constexpr int MINW = 2; };
template <> struct BwdTile<128> { static constexpr int BN = 32; static constexpr int MINW = 1; };

// The dK/dV stage keeps k, v and two accumulator sets per lane, so it streams narrower tiles.
template <int HS>
struct DkdvTile;
template <> struct DkdvTile<32> { static constexpr int BN = 64; static constexpr int MINW = 2; };
template <> struct DkdvTile<64> { static constexpr int BN = 32; static constexpr int MINW = 2; };
template <> struct DkdvTile<128> { static constexpr int BN = 32; static constexpr int MINW = 1; };

// Instruction order of a block of MFMAs (sched_group_barrier masks: 0x008 MFMA, 0x100 LDS
// read): N pairs of MFMAs, each pair followed by one LDS read while I < R.  Preceded by a group
// of reads, this keeps a fixed number of operand reads in flight ahead of the MFMAs.
template <int I, int N, int R>
__device__ __forceinline__ void pin_mfma_pairs() {
  if constexpr (I < N) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    if constexpr (I < R) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    pin_mfma_pairs<I + 1, N, R>();
  }
}

// ------------------------------------------------------------------------------------
// Stage 2: dQ.  Workgroup = 128 query rows; K/V tiles streamed through LDS.
// FORM_DELTA: the kernel forms delta = rowsum(O dO) from its own rows (O through strides so),
// with fa2_bwd_delta_kernel's products and summation order (the same bits), uses it and writes
// it for the dK/dV stage that follows; otherwise it reads delta.
template <int HS, bool CAUSAL, bool FORM_DELTA = false>
__global__ __launch_bounds__(256, BwdTile<HS>::MINW) void fa2_bwd_dq_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ Lg, float* __restrict__ delta,
    float* __restrict__ dQ, int nh, int T, int BH, int n_qtiles, RowStrides sq, RowStrides sk,
    RowStrides sv, RowStrides sdo, LStrides sl, RowStrides sdq, float scale, float scale_log2,
    const float* __restrict__ Og = nullptr, RowStrides so = {}, int heads_per_xcd = 0) {
  constexpr int BN = BwdTile<HS>::BN;
  constexpr int BM = 128;
  constexpr int H2 = HS / 2;
  constexpr int KP = HS + 4;  // both K and V rows are read as 16-byte row segments
  constexpr int TILE = BN * KP;
  constexpr int F4_ROW = HS / 4;
  constexpr int LOADS = BN * F4_ROW / 256;
  static_assert(BN * F4_ROW % 256 == 0, "tile must split evenly over 256 threads");
  __shared__ __attribute__((aligned(16))) float smem[2 * 2 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  // Head-major items over XCDs; causal items are query-tile pairs (n-1-p, p) of equal cost, or
  // (heads_per_xcd > 0) single query tiles longest first per XCD (lpt_tile).
  int bh, qa, qb = -1;  // the item's query tiles, in pass order (qb < 0: one pass)
  if (CAUSAL && heads_per_xcd > 0) {
    int rank;
    lpt_tile(blockIdx.x, heads_per_xcd, bh, rank);
    qa = n_qtiles - 1 - rank;
  } else {
    const int per_head = CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles;
    const int w = xcd_work_item(blockIdx.x, BH * per_head);
    if (w >= BH * per_head) return;
    bh = w / per_head;
    const int p = w - bh * per_head;
    qa = CAUSAL ? n_qtiles - 1 - p : p;
    if (CAUSAL && n_qtiles - 1 - p != p) qb = p;
  }
  const int b = bh / nh, h = bh - b * nh;

  const float* Kb = K + b * sk.b + h * sk.h;
  const float* Vb = V + b * sv.b + h * sv.h;

  const int n_pass = qb >= 0 ? 2 : 1;
  for (int pass = 0; pass < n_pass; ++pass) {
  const int qt = pass == 0 ? qa : qb;
  const int i0 = qt * BM + wave * 32;
  const int my_i = i0 + col;

  float qf[H2], dof[H2];
  float l2 = 0.0f, dl = 0.0f;  // L_i * log2(e) and delta_i of this lane's row
  float part[FORM_DELTA ? H2 / 4 : 1];  // delta's per-chunk products (FORM_DELTA)
  if (my_i < T) {
    const float* qp = Q + b * sq.b + h * sq.h + (int64_t)my_i * sq.t + half * H2;
    const float* gp = dO + b * sdo.b + h * sdo.h + (int64_t)my_i * sdo.t + half * H2;
#pragma unroll
    for (int c = 0; c < H2 / 4; ++c) {
      const float4 x = ld4(qp + 4 * c);
      const float4 g = ld4(gp + 4 * c);
      qf[4 * c + 0] = x.x; qf[4 * c + 1] = x.y; qf[4 * c + 2] = x.z; qf[4 * c + 3] = x.w;
      dof[4 * c + 0] = g.x; dof[4 * c + 1] = g.y; dof[4 * c + 2] = g.z; dof[4 * c + 3] = g.w;
    }
    l2 = Lg[b * sl.b + h * sl.h + (int64_t)my_i * sl.t] * kLog2e;
    if constexpr (FORM_DELTA) {
      // The delta kernel's per-float4 products (chunk c = half * H2/4 + u of the row), then its
      // xor tree over chunks: offset H2/4 pairs the two wave halves, the smaller ones chunks
      // u and u ^ off of this lane.
      const float* op = Og + b * so.b + h * so.h + (int64_t)my_i * so.t + half * H2;
#pragma unroll
      for (int c = 0; c < H2 / 4; ++c) {
        const float4 o = ld4(op + 4 * c);
        const float4 g = make_float4(dof[4 * c], dof[4 * c + 1], dof[4 * c + 2], dof[4 * c + 3]);
        part[c] = o.x * g.x + o.y * g.y + o.z * g.z + o.w * g.w;
      }
    } else {
      dl = delta[(int64_t)bh * T + my_i];
    }
  } else {
#pragma unroll
    for (int c = 0; c < H2; ++c) { qf[c] = 0.0f; dof[c] = 0.0f; }
  }
  if constexpr (FORM_DELTA) {
    // Rows past T: every chunk 0 (both halves take part in the exchange).
#pragma unroll
    for (int c = 0; c < H2 / 4; ++c) {
      if (my_i >= T) part[c] = 0.0f;
      part[c] = part[c] + xor32(part[c]);
    }
#pragma unroll
    for (int off = H2 / 8; off >= 1; off >>= 1)
#pragma unroll
      for (int c = 0; c < off; ++c) part[c] = part[c] + part[c + off];
    dl = part[0];
    if (my_i < T && half == 0) delta[(int64_t)bh * T + my_i] = dl;
  }

  f32x16 dqacc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) dqacc[d] = zero16();

  const int kv_end = CAUSAL ? min(T, (qt + 1) * BM) : T;
  const int n_stages = (kv_end + BN - 1) / BN;

  float4 kst[LOADS], vst[LOADS];
  // K/V rows of a stage through buffer resources over its valid rows: past T they read zero.
  auto gload = [&](int stage) {
    const int j0 = stage * BN;
    const int rows = min(BN, T - j0);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(Kb + (int64_t)j0 * sk.t, rows, sk.t, HS);
    const __amdgpu_buffer_rsrc_t rv = rows_rsrc(Vb + (int64_t)j0 * sv.t, rows, sv.t, HS);
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + 256 * u;
      const int r = f / F4_ROW, c4 = f % F4_ROW;
      kst[u] = ld4_buffer(rk, (r * (int)sk.t + 4 * c4) * 4);
      vst[u] = ld4_buffer(rv, (r * (int)sv.t + 4 * c4) * 4);
    }
  };
  auto lstore = [&](int buf) {
    float* ks = smem + buf * 2 * TILE;
    float* vs = ks + TILE;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + 256 * u;
      const int r = f / F4_ROW, c4 = f % F4_ROW;
      st4(ks + r * KP + 4 * c4, kst[u]);
      st4(vs + r * KP + 4 * c4, vst[u]);
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();

  for (int s = 0; s < n_stages; ++s) {
    const int buf = s & 1;
    if (s + 1 < n_stages) gload(s + 1);
    const float* ks = smem + buf * 2 * TILE;
    const float* vs = ks + TILE;

#pragma unroll
    for (int sub = 0; sub < BN / 32; ++sub) {
      const int jj0 = s * BN + sub * 32;
      if (jj0 >= T) continue;
      if (CAUSAL && jj0 > i0 + 31) continue;

      f32x16 sacc = zero16(), pacc = zero16();
      const float* krow = ks + (sub * 32 + col) * KP + half * H2;
      const float* vrow = vs + (sub * 32 + col) * KP + half * H2;
#pragma unroll
      for (int c = 0; c < H2 / 4; ++c) {
        const float4 kv = ld4(krow + 4 * c);
        const float4 vv = ld4(vrow + 4 * c);
        sacc = mfma32(kv.x, qf[4 * c + 0], sacc);
        pacc = mfma32(vv.x, dof[4 * c + 0], pacc);
        sacc = mfma32(kv.y, qf[4 * c + 1], sacc);
        pacc = mfma32(vv.y, dof[4 * c + 1], pacc);
        sacc = mfma32(kv.z, qf[4 * c + 2], sacc);
        pacc = mfma32(vv.z, dof[4 * c + 2], pacc);
        sacc = mfma32(kv.w, qf[4 * c + 3], sacc);
        pacc = mfma32(vv.w, dof[4 * c + 3], pacc);
      }

      const bool need_mask = (CAUSAL && jj0 + 31 > i0) || (jj0 + 32 > T);
      // dS^T (overwrites sacc): P (dP - delta), masked entries give exactly 0.
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(sacc[r], scale_log2, -l2));
        if (need_mask) {
          const int j = jj0 + mfma_row(r, half);
          if ((CAUSAL && j > my_i) || j >= T) p = 0.0f;
        }
        sacc[r] = p * (pacc[r] - dl);
      }

      // K^T operand (key row R(kk, half), column d*32 + col) from a lane base pointer.
      const float* kcol = ks + (sub * 32 + 4 * half) * KP + col;
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
        for (int d = 0; d < HS / 32; ++d)
          dqacc[d] = mfma32(kcol[(8 * (kk >> 2) + (kk & 3)) * KP + d * 32], sacc[kk], dqacc[d]);
      }
    }

    if (s + 1 < n_stages) lstore(buf ^ 1);
    __syncthreads();
  }

  if (my_i < T) {
    float* op = dQ + b * sdq.b + h * sdq.h + (int64_t)my_i * sdq.t;
#pragma unroll
    for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dc = d * 32 + 8 * g + 4 * half;
        st4(op + dc, make_float4(dqacc[d][4 * g + 0] * scale, dqacc[d][4 * g + 1] * scale,
                                 dqacc[d][4 * g + 2] * scale, dqacc[d][4 * g + 3] * scale));
      }
    }
  }
  }  // pass
}

// ------------------------------------------------------------------------------------
// Stored dS tiles (ds_tile_index, cta_common.hpp).  An FP32 tile holds its 1024 floats in the
// order of the wave that consumes it: lane l = 32*h + c reads float4 g at offset 256*g + 4*l,
// which holds dS[32*ib + c][32*jb + 8*g + 4*h + e] for e = 0..3 — the B operand of the
// 32x32x2 MFMA for contraction steps kk = 4*g + e.
constexpr int kDsTileFloats = 1024;
constexpr int kDsPitch = 40;  // LDS pitch of the per-wave transpose: halves 4 rows apart hit disjoint banks

// ------------------------------------------------------------------------------------
// Stage 3: dK, dV.  Workgroup = 32 * WAVES key rows (WAVES = 4, or 2 for short causal heads),
// each wave owning 32 of them and each lane one key row's
// k and v in registers.  Q, dO, L and delta stream through LDS in stages of BN query rows,
// copied global -> LDS directly (global_load_lds: no staging registers), double buffered,
// one barrier per stage.  Query rows past T are read clamped to row T-1 and masked to P = 0.
//
// The Q and dO tiles keep the padded pitch HS + 4, under which both access patterns are
// free of bank conflicts: the row-segment reads of the S / dP products and the column reads
// of the dV / dK products.  The async copies fill whole 1 KiB pieces of LDS per wave, so the
// lanes that land on pad words (or past the dO tile) copy a harmless in-bounds chunk there.
//
// Heads [bh_base, bh_base + BH) are processed; with STORE_DS every dS tile is also written
// to dsw (heads indexed from bh_base).  A dS tile goes to a per-wave LDS transpose buffer when
// it is formed and out to HBM at the start of the next stage, so its stores drain behind a
// stage of MFMAs rather than in front of the stage's vmcnt wait.
//
// FOLD: delta is not read from a delta stage's output but computed here, per query stage, from
// the stage's dO tile and an O tile streamed beside it (delta_i = O_i . dO_i, the reference's
// flash_attention_bwd_delta, flash_attention.cuh:175-213, folded in).  Every key tile of a head
// recomputes it, and the stage needs a second barrier before delta is read.
//
// SPLIT: each work item (key-tile pair, or tile) is run by two workgroups, part 0 and part 1,
// each over one half of the item's query stages (in the item's stage order, across its passes);
// every dS tile is still stored once, by the part that forms it.  Part 0 writes its partial dK
// and dV to dK / dV, part 1 densely to part_ws (dK, then dV, of all BH heads); zeros where a
// part saw no query stage.  fa2_bwd_dkdv_sum_kernel then adds part 1 to part 0.
template <int HS, bool CAUSAL, bool STORE_DS, bool FOLD, int WAVES = 4, bool SPLIT = false>
__global__ __launch_bounds__(64 * WAVES, DkdvTile<HS>::MINW) void fa2_bwd_dkdv_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ O, const float* __restrict__ Lg,
    const float* __restrict__ delta, float* __restrict__ dK, float* __restrict__ dV,
    float* __restrict__ dsw, int nh, int T, int bh_base, int BH, int n_ktiles, RowStrides sq,
    RowStrides sk, RowStrides sv, RowStrides sdo, RowStrides so, LStrides sl, RowStrides sdk,
    RowStrides sdv, float scale, float scale_log2, float* __restrict__ part_ws = nullptr,
    int heads_per_xcd = 0) {
  constexpr int BN = DkdvTile<HS>::BN;
  constexpr int NSUB = BN / 32;
  constexpr int THREADS = 64 * WAVES;
  constexpr int BM = 32 * WAVES;  // key rows per workgroup, 32 per wave
  constexpr int H2 = HS / 2;
  constexpr int KP = HS + 4;                // LDS pitch of a Q / dO row
  constexpr int PPT = (BN * KP + 255) / 256;  // 1 KiB async copies per tile
  constexpr int TILE = PPT * 256;           // a tile's LDS extent: whole copies, rows then pad
  constexpr int NT = FOLD ? 3 : 2;          // tiles per stage: Q, dO (and O when folding delta)
  constexpr int PIECES = NT * PPT;
  constexpr int QG = PIECES * 256;
  constexpr int RVEC = 64;                  // L and delta of a stage, padded to one wave
  constexpr int STAGE = QG + 2 * RVEC;
  constexpr int PER_WAVE = (PIECES + WAVES - 1) / WAVES;
  static_assert(BN <= RVEC, "one wave copies a stage's L and delta");
  constexpr int XPOSE = STORE_DS ? WAVES * NSUB * 32 * kDsPitch : 0;
  __shared__ __attribute__((aligned(16))) float smem[2 * STAGE + XPOSE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  // Head-major items over XCDs; causal items are key-tile pairs (p, n-1-p) of equal cost, or
  // (heads_per_xcd > 0, unsplit) single key tiles longest first per XCD (lpt_tile).
  int bh_local, part = 0;
  int ka, kb = -1;  // the item's key tiles, in pass order (kb < 0: one pass)
  if (CAUSAL && !SPLIT && heads_per_xcd > 0) {
    lpt_tile(blockIdx.x, heads_per_xcd, bh_local, ka);  // key tile 0 is the longest
  } else {
    const int per_head = CAUSAL ? (n_ktiles + 1) / 2 : n_ktiles;
    const int n_items = BH * per_head * (SPLIT ? 2 : 1);
    const int w = xcd_work_item(blockIdx.x, n_items);
    if (w >= n_items) return;
    const int item = SPLIT ? w >> 1 : w;
    part = SPLIT ? w & 1 : 0;  // the two parts of an item are neighbours: one XCD
    bh_local = item / per_head;
    const int p = item - bh_local * per_head;
    ka = p;
    if (CAUSAL && n_ktiles - 1 - p != p) kb = n_ktiles - 1 - p;
  }
  const int bh = bh_base + bh_local;
  const int b = bh / nh, h = bh - b * nh;

  const float* Qb = Q + b * sq.b + h * sq.h;
  const float* dOb = dO + b * sdo.b + h * sdo.h;
  const float* Ob = FOLD ? O + b * so.b + h * so.h : nullptr;
  const float* Lb = Lg + b * sl.b + h * sl.h;
  const float* Db = FOLD ? nullptr : delta + (int64_t)bh * T;
  const int nb = (T + 31) / 32;
  // Byte offset of each of this lane's copies within its tile's first row of a stage: copy pc
  // fills floats [256 (pc % PPT), +256) of tile pc / PPT, the lane 4 of them at row f / KP,
  // column f % KP.  Pad columns and rows past the tile are out of range (no bytes read).
  int voff[PER_WAVE];
#pragma unroll
  for (int u = 0; u < PER_WAVE; ++u) {
    const int pc = wave + WAVES * u;
    const int which = pc / PPT;
    const int f = (pc - which * PPT) * 256 + lane * 4;
    const int r = f / KP, c = f - r * KP;
    const int64_t st = which == 0 ? sq.t : (FOLD && which == 2) ? so.t : sdo.t;
    voff[u] = pc < PIECES && r < BN && c < HS ? (int)((r * st + c) * 4) : (int)0x80000000;
  }
  float* xpose = smem + 2 * STAGE + wave * NSUB * 32 * kDsPitch;  // this wave's dS buffers
  float* dsh = STORE_DS ? dsw + (int64_t)bh_local * ds_tiles_per_head(T, CAUSAL) * kDsTileFloats
                        : nullptr;

  // Both stage buffers start as zeros, so the rows and pad words no copy writes are finite.
#pragma unroll 4
  for (int e = 4 * tid; e < 2 * STAGE; e += 4 * THREADS) st4(smem + e, zero4());
  __syncthreads();

  const int n_pass = kb >= 0 ? 2 : 1;
  auto kt_of = [&](int pass) { return pass == 0 ? ka : kb; };
  const int n_stages = (T + BN - 1) / BN;
  // first query stage that can see the keys of tile kt
  auto q_begin_of = [&](int kt) { return CAUSAL ? (kt * BM / BN) : 0; };
  // SPLIT: this part's positions [g0, g1) in the item's list of steps (pass 0's, then pass 1's).
  int g0 = 0, g1 = 0, pos = 0;
  if constexpr (SPLIT) {
    int total = 0;
    for (int pass = 0; pass < n_pass; ++pass) total += n_stages - q_begin_of(kt_of(pass));
    g0 = part ? (total + 1) / 2 : 0;
    g1 = part ? total : (total + 1) / 2;
  }
  for (int pass = 0; pass < n_pass; ++pass) {
  const int kt = kt_of(pass);
  const int j0 = kt * BM + wave * 32;  // first key row of this wave
  const int my_j = j0 + col;

  float kf[H2], vf[H2];
  if (my_j < T) {
    const float* kp = K + b * sk.b + h * sk.h + (int64_t)my_j * sk.t + half * H2;
    const float* vp = V + b * sv.b + h * sv.h + (int64_t)my_j * sv.t + half * H2;
#pragma unroll
    for (int c = 0; c < H2 / 4; ++c) {
      const float4 x = ld4(kp + 4 * c);
      const float4 y = ld4(vp + 4 * c);
      kf[4 * c + 0] = x.x; kf[4 * c + 1] = x.y; kf[4 * c + 2] = x.z; kf[4 * c + 3] = x.w;
      vf[4 * c + 0] = y.x; vf[4 * c + 1] = y.y; vf[4 * c + 2] = y.z; vf[4 * c + 3] = y.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < H2; ++c) { kf[c] = 0.0f; vf[c] = 0.0f; }
  }

  f32x16 dkacc[HS / 32], dvacc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) { dkacc[d] = zero16(); dvacc[d] = zero16(); }

  const int q_begin = q_begin_of(kt);
  const bool wave_stores = STORE_DS && j0 < T;

  // Async copies of stage `stage` into buffer `buf`.  Piece pc covers floats
  // [256 pc, 256 pc + 256) of the Q|dO region; wave w copies pieces w, w + WAVES, ...
  // Each tile of a stage is read through a buffer resource over its valid rows (base and
  // extent are scalar), so the per-lane offsets above serve every stage; rows past T are out of
  // range and keep the zeros (or an earlier stage's rows) in LDS, masked to P = 0.
  auto issue = [&](int stage, int buf) {
    float* qs = smem + buf * STAGE;
    const int r0 = stage * BN;
    const int rows = min(BN, T - r0);
    auto rsrc = [&](const float* base, int64_t st) {
      return rows_rsrc(base + (int64_t)r0 * st, rows, st, HS);
    };
    const __amdgpu_buffer_rsrc_t rq = rsrc(Qb, sq.t), rg = rsrc(dOb, sdo.t);
    const __amdgpu_buffer_rsrc_t ro = FOLD ? rsrc(Ob, so.t) : rq;
#pragma unroll
    for (int u = 0; u < PER_WAVE; ++u) {
      const int pc = wave + WAVES * u;
      if (pc < PIECES) {
        const int which = pc / PPT;  // 0: Q, 1: dO, 2: O (FOLD)
        async_copy16_buffer(which == 0 ? rq : which == 1 ? rg : ro, voff[u], qs + pc * 256);
      }
    }
    if (wave == 0) {  // lanes past BN fill the padding
      const int64_t i = min(r0 + lane, T - 1);
      async_copy4(Lb + i * sl.t, qs + QG);
      if (!FOLD) async_copy4(Db + i, qs + QG + RVEC);
    }
  };
  // FOLD: delta of the stage in buffer `st` from its O and dO tiles, THREADS / BN lanes per row,
  // into the stage's delta slot.  Rows past T hold row T - 1 (their P is masked to 0).
  auto fold_delta = [&](float* st) {
    constexpr int LPR = THREADS / BN;  // lanes per row (consecutive lanes of one wave)
    constexpr int DPL = HS / LPR;      // d values per lane
    static_assert(THREADS % BN == 0 && DPL % 4 == 0 && LPR <= 64, "delta split");
    const int r = tid / LPR, seg = tid % LPR;
    const float* orow = st + 2 * TILE + r * KP + seg * DPL;
    const float* grow = st + TILE + r * KP + seg * DPL;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < DPL / 4; ++c) {
      const float4 o4 = ld4(orow + 4 * c), g4 = ld4(grow + 4 * c);
      acc = fmaf(o4.x, g4.x, acc);
      acc = fmaf(o4.y, g4.y, acc);
      acc = fmaf(o4.z, g4.z, acc);
      acc = fmaf(o4.w, g4.w, acc);
    }
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
    if (seg == 0) st[QG + RVEC + r] = acc;
  };
  // Tiles whose every query row precedes every key row are skipped (dS = 0, nothing stored).
  auto live = [&](int ii0) { return ii0 < T && !(CAUSAL && ii0 + 31 < j0); };
  // Copy the dS tiles of `stage` from the transpose buffers to the workspace.
  auto flush = [&](int stage) {
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int ii0 = stage * BN + sub * 32;
      if (!live(ii0)) continue;
      const float* xw = xpose + sub * 32 * kDsPitch;
      float* gt = dsh + ds_tile_index(ii0 / 32, j0 / 32, nb, CAUSAL) * kDsTileFloats;
      wave_lds_fence();
#pragma unroll
      for (int g = 0; g < 4; ++g)
        st4_stream(gt + 256 * g + 4 * lane, ld4(xw + col * kDsPitch + 8 * g + 4 * half));
      wave_lds_fence();
    }
  };

  // Stage order.  With a causal mask the first (long) pass walks its query stages downward
  // from the last and the second (short) pass upward from its first, so every workgroup of a
  // head in its first pass reads query stage n-1-t at step t and every one in its second pass
  // reads stage t - 4 (t counted from the item's start): the workgroups of a head share each
  // streamed Q / dO stage in L2 instead of each reading it at a different time.
  const int n_steps = n_stages - q_begin;
  // the steps [i_begin, i_end) of this pass that this part runs (all of them unless SPLIT)
  const int i_begin = SPLIT ? min(max(g0 - pos, 0), n_steps) : 0;
  const int i_end = SPLIT ? min(max(g1 - pos, 0), n_steps) : n_steps;
  pos += n_steps;
  // (the long tile of a pair walks down: a property of the tile, so single tiles match pairs)
  const bool down = CAUSAL && kt <= n_ktiles - 1 - kt;
  auto stage_at = [&](int i) { return down ? n_stages - 1 - i : q_begin + i; };
  if (i_begin < i_end) issue(stage_at(i_begin), 0);
  vm_wait_all();
  __syncthreads();

  for (int i = i_begin; i < i_end; ++i) {
    const int s = stage_at(i);
    const int buf = (i - i_begin) & 1;
    if (i + 1 < i_end) issue(stage_at(i + 1), buf ^ 1);
    if (wave_stores && i > i_begin) flush(stage_at(i - 1));
    if (FOLD) {
      fold_delta(smem + buf * STAGE);
      __syncthreads();
    }
    const float* qs = smem + buf * STAGE;
    const float* gs = qs + TILE;
    const float* ls = qs + QG;
    const float* ds = ls + RVEC;

#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int ii0 = s * BN + sub * 32;
      if (!live(ii0)) continue;

      // S and dP tiles: lane holds column my_j, rows ii0 + R(r, half)
      f32x16 sacc = zero16(), pacc = zero16();
      const float* qrow = qs + (sub * 32 + col) * KP + half * H2;
      const float* grow = gs + (sub * 32 + col) * KP + half * H2;
#pragma unroll
      for (int c = 0; c < H2 / 4; ++c) {
        const float4 qv = ld4(qrow + 4 * c);
        const float4 gv = ld4(grow + 4 * c);
        sacc = mfma32(qv.x, kf[4 * c + 0], sacc);
        pacc = mfma32(gv.x, vf[4 * c + 0], pacc);
        sacc = mfma32(qv.y, kf[4 * c + 1], sacc);
        pacc = mfma32(gv.y, vf[4 * c + 1], pacc);
        sacc = mfma32(qv.z, kf[4 * c + 2], sacc);
        pacc = mfma32(gv.z, vf[4 * c + 2], pacc);
        sacc = mfma32(qv.w, kf[4 * c + 3], sacc);
        pacc = mfma32(gv.w, vf[4 * c + 3], pacc);
      }

      // Masked entries (and, when storing dS, key rows past T, so a stored tile is exactly 0
      // there) become -inf, so P = 2^-inf = 0 below.  A separate block behind a wave-uniform
      // branch: inside the exponential loop the test is if-converted into per-element
      // predication that every tile pays for.
      if ((CAUSAL && ii0 < j0 + 31) || (ii0 + 32 > T) || (STORE_DS && j0 + 32 > T)) {
        asm volatile("");  // a side effect keeps the block from being speculated into selects
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = ii0 + mfma_row(r, half);
          if ((CAUSAL && my_j > i) || i >= T || (STORE_DS && my_j >= T)) sacc[r] = -INFINITY;
        }
      }
      // P = e^{S - L}; masked entries are exactly 0.
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 lv = ld4(ls + sub * 32 + 8 * g + 4 * half);
        const float lr[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          sacc[r] = fast_exp2(fmaf(sacc[r], scale_log2, -lr[e] * kLog2e));
        }
      }

      // dV^T += dO^T P is issued before dS is formed, so the dS arithmetic and its transpose
      // writes overlap these MFMAs; then dK^T += Q^T dS.  One product at a time keeps at most
      // one set of LDS operands in flight.
      //
      // The A operand of step kk is (query row R(kk, half), column d*32 + col) of the dO or Q
      // tile.  For HS <= 64 it is addressed from one lane base pointer plus a compile-time row
      // offset (8 (kk/4) + kk%4), which the LDS reads carry as immediates: per-read row
      // arithmetic held registers at the 256-VGPR limit and forced each read to wait just
      // before its MFMA.  With the registers free, the reads are pinned several MFMA pairs
      // ahead.  HS = 128 (one wave per SIMD) measured faster with the per-read form.
      const float* gcol = gs + (sub * 32 + 4 * half) * KP + col;
      const float* qcol = qs + (sub * 32 + 4 * half) * KP + col;
      auto a_op = [&](const float* tile, const float* lane_col, int kk, int d) {
        return HS == 128 ? tile[(sub * 32 + mfma_row(kk, half)) * KP + d * 32 + col]
                         : lane_col[(8 * (kk >> 2) + (kk & 3)) * KP + d * 32];
      };
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
        for (int d = 0; d < HS / 32; ++d) dvacc[d] = mfma32(a_op(gs, gcol, kk, d), sacc[kk], dvacc[d]);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 dv = ld4(ds + sub * 32 + 8 * g + 4 * half);
        const float dr[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) pacc[4 * g + e] = sacc[4 * g + e] * (pacc[4 * g + e] - dr[e]);
      }
      // L's four reads and four dO pairs ahead of the first MFMA pair, then one read (dO
      // operands, then delta) after each pair.
      if (HS == 64) {
        __builtin_amdgcn_sched_group_barrier(0x100, 4 + 4, 0);
        pin_mfma_pairs<0, 16, 16>();
      }

      // Lane (col, half) holds dS[ii0 + R(r, half)][j0 + col]: into the transpose buffer as
      // [query][key]; flush() reads it back one query row per lane.  A wave's LDS operations
      // complete in order, so no barrier separates the write, the read and the next write.
      if (wave_stores) {
        float* xw = xpose + sub * 32 * kDsPitch;
#pragma unroll
        for (int r = 0; r < 16; ++r) xw[mfma_row(r, half) * kDsPitch + col] = pacc[r];
      }

#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
        for (int d = 0; d < HS / 32; ++d) dkacc[d] = mfma32(a_op(qs, qcol, kk, d), pacc[kk], dkacc[d]);
      }
      if (HS == 64) {  // four Q pairs ahead
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        pin_mfma_pairs<0, 16, 12>();
      }
    }

    vm_wait_all();
    __syncthreads();
  }
  if (wave_stores && i_end > i_begin) flush(stage_at(i_end - 1));

  if (my_j < T) {
    float* kp = dK + b * sdk.b + h * sdk.h + (int64_t)my_j * sdk.t;
    float* vp = dV + b * sdv.b + h * sdv.h + (int64_t)my_j * sdv.t;
    if (SPLIT && part) {
      kp = part_ws + ((int64_t)bh * T + my_j) * HS;
      vp = kp + (int64_t)(bh_base + BH) * T * HS;
    }
#pragma unroll
    for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dc = d * 32 + 8 * g + 4 * half;
        st4(kp + dc, make_float4(dkacc[d][4 * g + 0] * scale, dkacc[d][4 * g + 1] * scale,
                                 dkacc[d][4 * g + 2] * scale, dkacc[d][4 * g + 3] * scale));
        st4(vp + dc, make_float4(dvacc[d][4 * g + 0], dvacc[d][4 * g + 1], dvacc[d][4 * g + 2],
                                 dvacc[d][4 * g + 3]));
      }
    }
  }
  }  // pass: the stage loop ended on a barrier, so the next pass may refill LDS
}

// dK += part 1's dK, dV += part 1's dV, row by row in a fixed order (part 0, then part 1), after
// a split dK/dV stage; dK / dV through their strides, part 1 dense in part_ws.  HS / 4 lanes
// per row, one float4 each.
template <int HS>
__global__ __launch_bounds__(256) void fa2_bwd_dkdv_sum_kernel(float* __restrict__ dK,
                                                               float* __restrict__ dV,
                                                               const float* __restrict__ part_ws,
                                                               int nh, int T, int64_t rows,
                                                               RowStrides sdk, RowStrides sdv) {
  constexpr int G = HS / 4;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / G;
  if (row >= rows) return;
  const int c4 = (int)(gid % G);
  const int64_t bh = row / T;
  const int t = (int)(row - bh * T);
  const int64_t b = bh / nh, h = bh - b * nh;
  float* kp = dK + b * sdk.b + h * sdk.h + (int64_t)t * sdk.t + 4 * c4;
  float* vp = dV + b * sdv.b + h * sdv.h + (int64_t)t * sdv.t + 4 * c4;
  const float4 a = ld4(kp), c = ld4(part_ws + row * HS + 4 * c4);
  const float4 x = ld4(vp), y = ld4(part_ws + (rows + row) * HS + 4 * c4);
  st4(kp, make_float4(a.x + c.x, a.y + c.y, a.z + c.z, a.w + c.w));
  st4(vp, make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
}

// dQ += part 1's dQ, row by row (part 0, then part 1), after a split dQ-from-dS stage; dQ
// through its strides, part 1 dense in part_ws.  HS / 4 lanes per row, one float4 each.
template <int HS>
__global__ __launch_bounds__(256) void fa2_bwd_dq_sum_kernel(float* __restrict__ dQ,
                                                             const float* __restrict__ part_ws,
                                                             int nh, int T, int64_t rows,
                                                             RowStrides sdq) {
  constexpr int G = HS / 4;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / G;
  if (row >= rows) return;
  const int c4 = (int)(gid % G);
  const int64_t bh = row / T;
  const int t = (int)(row - bh * T);
  const int64_t b = bh / nh, h = bh - b * nh;
  float* qp = dQ + b * sdq.b + h * sdq.h + (int64_t)t * sdq.t + 4 * c4;
  const float4 a = ld4(qp), c = ld4(part_ws + row * HS + 4 * c4);
  st4(qp, make_float4(a.x + c.x, a.y + c.y, a.z + c.z, a.w + c.w));
}

// ------------------------------------------------------------------------------------
// dQ from stored dS tiles: dQ^T += K^T dS^T, one 32x32 tile per MFMA chain.  Workgroup =
// 32 * WAVES query rows (WAVES = 4, or 2 for short causal heads).  K tiles of 64 rows go
// global -> registers -> LDS, double
// buffered; each wave streams its own dS tiles from the workspace straight into registers,
// one stage ahead, as the B operand.  Heads [bh_base, bh_base + BH).
// SPLIT (small grids, heads from 0): each item's key stages (pass 0's, then pass 1's) are
// split over two workgroups, neighbours in the XCD order; part 0 writes dQ, part 1 its
// partial dQ densely into part_ws, and fa2_bwd_dq_sum_kernel adds the two in that order.
__device__ __forceinline__ float f4_at(const float4& v, int e) {
  return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

template <int HS, bool CAUSAL, int WAVES = 4, bool SPLIT = false>
__global__ __launch_bounds__(64 * WAVES, 2) void fa2_bwd_dq_ds_kernel(
    const float* __restrict__ K, const float* __restrict__ dsw, float* __restrict__ dQ, int nh,
    int T, int bh_base, int BH, int n_qtiles, RowStrides sk, RowStrides sdq, float scale,
    float* __restrict__ part_ws = nullptr, int heads_per_xcd = 0) {
  constexpr int BN = 64;
  constexpr int NSUB = BN / 32;
  constexpr int THREADS = 64 * WAVES;
  constexpr int BM = 32 * WAVES;  // query rows per workgroup, 32 per wave
  constexpr int KP = HS + 8;  // column reads of rows R(kk, 0) and R(kk, 1) = +4: disjoint banks
  constexpr int TILE = BN * KP;
  constexpr int F4_ROW = HS / 4;
  constexpr int LOADS = BN * F4_ROW / THREADS;
  static_assert(BN * F4_ROW % THREADS == 0, "tile must split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) float smem[2 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  // Head-major items over XCDs; causal items are query-tile pairs (n-1-p, p) of equal cost, or
  // (heads_per_xcd > 0, unsplit) single query tiles longest first per XCD (lpt_tile).
  int bh_local, part = 0;
  int qa, qb = -1;  // the item's query tiles, in pass order (qb < 0: one pass)
  if (CAUSAL && !SPLIT && heads_per_xcd > 0) {
    int rank;
    lpt_tile(blockIdx.x, heads_per_xcd, bh_local, rank);
    qa = n_qtiles - 1 - rank;
  } else {
    const int per_head = CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles;
    const int n_items = BH * per_head * (SPLIT ? 2 : 1);
    const int w = xcd_work_item(blockIdx.x, n_items);
    if (w >= n_items) return;
    const int item = SPLIT ? w >> 1 : w;
    part = SPLIT ? w & 1 : 0;
    bh_local = item / per_head;
    const int p = item - bh_local * per_head;
    qa = CAUSAL ? n_qtiles - 1 - p : p;
    if (CAUSAL && n_qtiles - 1 - p != p) qb = p;
  }
  const int bh = bh_base + bh_local;
  const int b = bh / nh, h = bh - b * nh;
  const float* Kb = K + b * sk.b + h * sk.h;
  const int nb = (T + 31) / 32;
  const float* dsh = dsw + (int64_t)bh_local * ds_tiles_per_head(T, CAUSAL) * kDsTileFloats;

  const int n_pass = qb >= 0 ? 2 : 1;
  auto qt_of = [&](int pass) { return pass == 0 ? qa : qb; };
  auto stages_of = [&](int qt) {
    const int kv_end = CAUSAL ? min(T, (qt + 1) * BM) : T;
    return (kv_end + BN - 1) / BN;
  };
  // SPLIT: this part's positions [g0, g1) in the item's list of stages (pass 0's, then pass 1's).
  int g0 = 0, g1 = 0, pos = 0;
  if constexpr (SPLIT) {
    int total = 0;
    for (int pass = 0; pass < n_pass; ++pass) total += stages_of(qt_of(pass));
    g0 = part ? (total + 1) / 2 : 0;
    g1 = part ? total : (total + 1) / 2;
  }
  for (int pass = 0; pass < n_pass; ++pass) {
  const int qt = qt_of(pass);
  const int i0 = qt * BM + wave * 32;
  const int my_i = i0 + col;
  const int ib = i0 / 32;  // query block of this wave

  f32x16 acc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) acc[d] = zero16();

  const int n_stages = stages_of(qt);
  // the stages [s_begin, s_end) of this pass that this part runs (all of them unless SPLIT)
  const int s_begin = SPLIT ? min(max(g0 - pos, 0), n_stages) : 0;
  const int s_end = SPLIT ? min(max(g1 - pos, 0), n_stages) : n_stages;
  pos += n_stages;

  // Every stage issues the same loads, unconditionally (K through a buffer resource, dS from
  // clamped in-bounds tiles), and the stage count is padded to even (padded stages compute
  // nothing).  The compiler can then
  // count the loads in flight exactly: the MFMAs of stage s wait only for stage s's dS, not
  // for the stage s+1 loads issued ahead of them.
  float4 kst[LOADS];
  // K rows through a buffer resource over the stage's valid rows (none for a padded stage):
  // keys past T read as zero, as they must, since they meet finite dS columns.
  auto gload = [&](int stage) {
    const int j0 = stage * BN;
    const int rows = min(BN, T - j0);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc(Kb + (int64_t)j0 * sk.t, rows, sk.t, HS);
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + THREADS * u;
      const int r = f / F4_ROW, c4 = f % F4_ROW;
      kst[u] = ld4_buffer(rk, (r * (int)sk.t + 4 * c4) * 4);
    }
  };
  auto lstore = [&](int buf) {
    float* ks = smem + buf * TILE;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + THREADS * u;
      const int r = f / F4_ROW, c4 = f % F4_ROW;
      st4(ks + r * KP + 4 * c4, kst[u]);
    }
  };
  // A stored tile exists for query block ib and key block jb iff both lie inside the head and,
  // with a causal mask, jb <= ib (the wave-uniform skip of the dK/dV stage).
  auto has_tile = [&](int jb) { return ib < nb && jb < nb && (!CAUSAL || jb <= ib); };
  // Tiles that do not exist are read from the row's last stored tile (clamped block indices,
  // equal to (ib, jb) whenever has_tile(jb)); compute() skips them.
  const int ibc = min(ib, nb - 1);
  auto dsload = [&](int stage, float4 (&dr)[NSUB][4]) {
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int jbc = min(stage * NSUB + sub, CAUSAL ? ibc : nb - 1);
      const float* src = dsh + ds_tile_index(ibc, jbc, nb, CAUSAL) * kDsTileFloats + 4 * lane;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        dr[sub][g] = ld4_stream(src + 256 * g);
      }
    }
  };
  auto compute = [&](int stage, const float* ks, const float4 (&dr)[NSUB][4]) {
    if (stage >= s_end) return;  // a padded stage (or, split, the other part's)
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      if (!has_tile(stage * NSUB + sub)) continue;
      // kk-major: the HS/32 accumulator chains alternate, so no MFMA waits on its predecessor
      // K^T operand (key row R(kk, half), column d*32 + col): lane base pointer plus
      // compile-time row offsets, carried by the LDS reads as immediates.
      const float* kcol = ks + (sub * 32 + 4 * half) * KP + col;
#pragma unroll
      for (int kk = 0; kk < 16; ++kk) {
#pragma unroll
        for (int d = 0; d < HS / 32; ++d)
          acc[d] = mfma32(kcol[(8 * (kk >> 2) + (kk & 3)) * KP + d * 32],
                          f4_at(dr[sub][kk >> 2], kk & 3), acc[d]);
      }
    }
  };
  auto step = [&](int s, const float4 (&cur)[NSUB][4], float4 (&nxt)[NSUB][4]) {
    const int buf = (s - s_begin) & 1;
    gload(s + 1);
    dsload(s + 1, nxt);
    compute(s, smem + buf * TILE, cur);
    lstore(buf ^ 1);
    __syncthreads();
  };

  if (s_end > s_begin) {
    float4 dA[NSUB][4], dB[NSUB][4];
    dsload(s_begin, dA);
    gload(s_begin);
    lstore(0);
    __syncthreads();
    // Unrolled by two so the two dS register sets swap roles without copies.
    const int n_run2 = (s_end - s_begin + 1) & ~1;
    for (int s = s_begin; s < s_begin + n_run2; s += 2) {
      step(s, dA, dB);
      step(s + 1, dB, dA);
    }
  }

  if (my_i < T) {
    float* op = dQ + b * sdq.b + h * sdq.h + (int64_t)my_i * sdq.t;
    if (SPLIT && part) op = part_ws + ((int64_t)bh * T + my_i) * HS;
#pragma unroll
    for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dc = d * 32 + 8 * g + 4 * half;
        st4(op + dc, make_float4(acc[d][4 * g + 0] * scale, acc[d][4 * g + 1] * scale,
                                 acc[d][4 * g + 2] * scale, acc[d][4 * g + 3] * scale));
      }
    }
  }
  }  // pass: the stage loop ended on a barrier, so the next pass may refill LDS
}

RowStrides rs(const int64_t* s) { return RowStrides{s[0], s[1], s[2]}; }

template <int HS>
void launch_delta(const float* o, const float* d_o, float* delta, int nh, int T, int64_t rows,
                  RowStrides so, RowStrides sdo, hipStream_t st) {
  const int64_t threads = rows * (HS / 4);
  const unsigned grid = (unsigned)((threads + 255) / 256);
  hipLaunchKernelGGL((fa2_bwd_delta_kernel<HS>), dim3(grid), dim3(256), 0, st, o, d_o, delta, nh,
                     T, rows, so, sdo);
}

// With o != nullptr the kernel forms delta from O (strides so) and writes it into `delta`.
template <int HS, bool CAUSAL>
void launch_dq(const float* q, const float* k, const float* v, const float* d_o, const float* l,
               float* delta, float* dq, int nh, int T, int BH, RowStrides sq,
               RowStrides sk, RowStrides sv, RowStrides sdo, LStrides sl, RowStrides sdq,
               float scale, hipStream_t st, const float* o = nullptr, RowStrides so = {}) {
  const int n_qtiles = (T + 127) / 128;
  const int64_t items = (int64_t)(CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles) * BH;
  const int lpt = CAUSAL ? lpt_heads(BH, n_qtiles, 4, BwdTile<HS>::MINW) : 0;
  const dim3 grid(lpt > 0 ? (unsigned)(BH * n_qtiles) : xcd_grid(items));
  if (o != nullptr) {
    hipLaunchKernelGGL((fa2_bwd_dq_kernel<HS, CAUSAL, true>), grid, dim3(256), 0, st, q, k, v,
                       d_o, l, delta, dq, nh, T, BH, n_qtiles, sq, sk, sv, sdo, sl, sdq, scale,
                       scale * kLog2e, o, so, lpt);
    return;
  }
  hipLaunchKernelGGL((fa2_bwd_dq_kernel<HS, CAUSAL>), grid, dim3(256), 0, st, q, k, v, d_o, l,
                     delta, dq, nh, T, BH, n_qtiles, sq, sk, sv, sdo, sl, sdq, scale,
                     scale * kLog2e, nullptr, RowStrides{}, lpt);
}

// dK/dV for heads [bh_base, bh_base + n_heads), written through strides sdk / sdv; with
// STORE_DS the dS tiles go to dsw; with FOLD delta comes from O (strides so) instead of the
// delta array.  Four waves (128 keys) per workgroup, or two for short causal heads.
// part_ws (heads [0, n_heads) with bh_base = 0 only): run the split form and its sum pass.
template <int HS, bool CAUSAL, bool STORE_DS, bool FOLD = false>
void launch_dkdv(const float* q, const float* k, const float* v, const float* d_o,
                 const float* l, const float* delta, float* dk, float* dv, float* dsw, int nh,
                 int T, int bh_base, int n_heads, RowStrides sq, RowStrides sk, RowStrides sv,
                 RowStrides sdo, LStrides sl, RowStrides sdk, RowStrides sdv, float scale,
                 hipStream_t st, const float* o = nullptr, RowStrides so = {},
                 float* part_ws = nullptr) {
  auto run = [&]<int WAVES>() {
    const int n_ktiles = (T + 32 * WAVES - 1) / (32 * WAVES);
    const int64_t items = (int64_t)(CAUSAL ? (n_ktiles + 1) / 2 : n_ktiles) * n_heads;
    if (part_ws != nullptr) {
      hipLaunchKernelGGL((fa2_bwd_dkdv_kernel<HS, CAUSAL, STORE_DS, FOLD, WAVES, true>),
                         dim3(xcd_grid(2 * items)), dim3(64 * WAVES), 0, st, q, k, v, d_o, o, l,
                         delta, dk, dv, dsw, nh, T, bh_base, n_heads, n_ktiles, sq, sk, sv, sdo,
                         so, sl, sdk, sdv, scale, scale * kLog2e, part_ws);
      const int64_t rows = (int64_t)n_heads * T;
      hipLaunchKernelGGL((fa2_bwd_dkdv_sum_kernel<HS>),
                         dim3((unsigned)((rows * (HS / 4) + 255) / 256)), dim3(256), 0, st, dk,
                         dv, part_ws, nh, T, rows, sdk, sdv);
      return;
    }
    const int lpt = CAUSAL ? lpt_heads(n_heads, n_ktiles, WAVES, DkdvTile<HS>::MINW) : 0;
    hipLaunchKernelGGL((fa2_bwd_dkdv_kernel<HS, CAUSAL, STORE_DS, FOLD, WAVES>),
                       dim3(lpt > 0 ? (unsigned)(n_heads * n_ktiles) : xcd_grid(items)),
                       dim3(64 * WAVES), 0, st, q, k, v, d_o, o, l, delta, dk, dv, dsw, nh, T,
                       bh_base, n_heads, n_ktiles, sq, sk, sv, sdo, so, sl, sdk, sdv, scale,
                       scale * kLog2e, nullptr, lpt);
  };
  // Short causal heads (hs 64, T <= 1024) run two waves (64 keys) per workgroup: the half-empty
  // diagonal blocks idle fewer waves at each stage's barrier and the pairs balance over more,
  // smaller workgroups.  A/B in one process: +17% at T = 256 (the GPT step's shape), +11% at
  // 512, +4% at 1024, equal at 2048; 26% slower non-causal at 256 and 39% at config 2, where
  // each key now costs twice the Q / dO staging.  Every schedule (stored dS, recompute, delta
  // folded) takes the same shape, so their dK / dV stay bitwise equal.
  if constexpr (HS == 64 && CAUSAL) {
    if (T <= 1024) {
      run.template operator()<2>();
      return;
    }
  }
  run.template operator()<4>();
}

// part_ws (heads [0, n_heads) with bh_base = 0 only): run the split form and its sum pass.
template <int HS, bool CAUSAL>
void launch_dq_ds(const float* k, const float* dsw, float* dq, int nh, int T, int bh_base,
                  int n_heads, RowStrides sk, RowStrides sdq, float scale, hipStream_t st,
                  float* part_ws = nullptr) {
  auto run = [&]<int WAVES>() {
    const int n_qtiles = (T + 32 * WAVES - 1) / (32 * WAVES);
    const int64_t items = (int64_t)(CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles) * n_heads;
    if (part_ws != nullptr) {
      hipLaunchKernelGGL((fa2_bwd_dq_ds_kernel<HS, CAUSAL, WAVES, true>),
                         dim3(xcd_grid(2 * items)), dim3(64 * WAVES), 0, st, k, dsw, dq, nh, T,
                         bh_base, n_heads, n_qtiles, sk, sdq, scale, part_ws);
      const int64_t rows = (int64_t)n_heads * T;
      hipLaunchKernelGGL((fa2_bwd_dq_sum_kernel<HS>),
                         dim3((unsigned)((rows * (HS / 4) + 255) / 256)), dim3(256), 0, st, dq,
                         part_ws, nh, T, rows, sdq);
      return;
    }
    const int lpt = CAUSAL ? lpt_heads(n_heads, n_qtiles, WAVES, 2) : 0;
    hipLaunchKernelGGL((fa2_bwd_dq_ds_kernel<HS, CAUSAL, WAVES>),
                       dim3(lpt > 0 ? (unsigned)(n_heads * n_qtiles) : xcd_grid(items)),
                       dim3(64 * WAVES), 0, st, k, dsw, dq, nh, T, bh_base, n_heads, n_qtiles, sk,
                       sdq, scale, nullptr, lpt);
  };
  // Short causal heads (hs 64, T <= 1024): two waves (64 query rows) per workgroup, as in the
  // dK/dV stage.  A/B in one process, bitwise-equal dQ: +11.5% at T = 256, +10% at 512, +5% at
  // 1024 (B16 H6), +0.5% at B4 H32 T1024.
  if constexpr (HS == 64 && CAUSAL) {
    if (T <= 1024) {
      run.template operator()<2>();
      return;
    }
  }
  run.template operator()<4>();
}

// The stored-dS dK/dV stage splits each item's query stages over two workgroups when its grid
// would hold fewer than two waves per SIMD (1024 SIMDs) and a full column of queries gives each
// part at least kSplitMinStages stages (T >= 1024 at 32-row stages), as the forward does.
constexpr int kSimds = 1024;
constexpr int kSplitMinStages = 16;

template <int HS, bool CAUSAL>
bool dkdv_split(int T, int BH) {
  const int waves = (HS == 64 && CAUSAL && T <= 1024) ? 2 : 4;
  const int n_ktiles = (T + 32 * waves - 1) / (32 * waves);
  const int64_t items = (int64_t)(CAUSAL ? (n_ktiles + 1) / 2 : n_ktiles) * BH;
  return items * waves < 2 * kSimds && T / DkdvTile<HS>::BN >= 2 * kSplitMinStages;
}

// Runs f.template operator()<HS, CAUSAL>() for the runtime head size and mask flag.
template <typename F>
void dispatch_hs_causal(int64_t hs, int causal, F&& f) {
  if (hs == 32) { if (causal) f.template operator()<32, true>(); else f.template operator()<32, false>(); }
  else if (hs == 64) { if (causal) f.template operator()<64, true>(); else f.template operator()<64, false>(); }
  else { if (causal) f.template operator()<128, true>(); else f.template operator()<128, false>(); }
}

bool l_ok(const float* l, const int64_t* s) { return l != nullptr && s != nullptr; }

}  // namespace
}  // namespace cta

using namespace cta;

extern "C" int cta_flash_attention_bwd_delta(const float* o, const int64_t* o_strides,
                                             const float* d_o, const int64_t* do_strides,
                                             int64_t B, int64_t nh, int64_t T, int64_t hs,
                                             float* delta, void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (!delta) return fail(CTA_ERR_INVALID_ARGUMENT, "null delta pointer");
  if (!attn_layout_ok(o, o_strides) || !attn_layout_ok(d_o, do_strides))
    return fail(CTA_ERR_LAYOUT,
                "flash_attention_bwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                "aligned O/dO");
  const int64_t rows = B * nh * T;
  hipStream_t st = as_stream(stream);
  if (hs == 32) launch_delta<32>(o, d_o, delta, (int)nh, (int)T, rows, rs(o_strides), rs(do_strides), st);
  else if (hs == 64) launch_delta<64>(o, d_o, delta, (int)nh, (int)T, rows, rs(o_strides), rs(do_strides), st);
  else launch_delta<128>(o, d_o, delta, (int)nh, (int)T, rows, rs(o_strides), rs(do_strides), st);
  return check_launch("flash_attention_bwd_delta");
}

namespace {
int check_bwd_inputs(const float* q, const int64_t* qs, const float* k, const int64_t* ks,
                     const float* v, const int64_t* vs, const float* d_o, const int64_t* dos,
                     const float* l, const int64_t* ls, const float* delta) {
  if (!attn_layout_ok(q, qs) || !attn_layout_ok(k, ks) || !attn_layout_ok(v, vs) ||
      !attn_layout_ok(d_o, dos))
    return fail(CTA_ERR_LAYOUT,
                "flash_attention_bwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                "aligned Q/K/V/dO");
  if (!l_ok(l, ls) || !delta) return fail(CTA_ERR_INVALID_ARGUMENT, "null L or delta pointer");
  return CTA_OK;
}
}  // namespace

namespace {
// Strides of a dense (B, nh, T, hs) output.
RowStrides dense_out(int64_t nh, int64_t T, int64_t hs) { return {nh * T * hs, T * hs, hs}; }

// With o != nullptr, dQ forms delta itself (from O, strides so) and writes it into `delta`.
int bwd_dq_impl(const float* q, const int64_t* q_strides, const float* k,
                const int64_t* k_strides, const float* v, const int64_t* v_strides,
                const float* d_o, const int64_t* do_strides, const float* l,
                const int64_t* l_strides, float* delta, int64_t B, int64_t nh, int64_t T,
                int64_t hs, int causal, float* dq, RowStrides sdq, hipStream_t st,
                const float* o = nullptr, RowStrides so = {}) {
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const LStrides sl{l_strides[0], l_strides[1], l_strides[2]};
  const int BH = (int)(B * nh);
  dispatch_hs_causal(hs, causal, [&]<int HS, bool C>() {
    launch_dq<HS, C>(q, k, v, d_o, l, delta, dq, (int)nh, (int)T, BH, rs(q_strides),
                     rs(k_strides), rs(v_strides), rs(do_strides), sl, sdq, scale, st, o, so);
  });
  return check_launch("flash_attention_bwd_dq");
}

int bwd_dkdv_impl(const float* q, const int64_t* q_strides, const float* k,
                  const int64_t* k_strides, const float* v, const int64_t* v_strides,
                  const float* d_o, const int64_t* do_strides, const float* l,
                  const int64_t* l_strides, const float* delta, int64_t B, int64_t nh, int64_t T,
                  int64_t hs, int causal, float* dk, RowStrides sdk, float* dv, RowStrides sdv,
                  hipStream_t st) {
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const LStrides sl{l_strides[0], l_strides[1], l_strides[2]};
  const int BH = (int)(B * nh);
  dispatch_hs_causal(hs, causal, [&]<int HS, bool C>() {
    launch_dkdv<HS, C, false>(q, k, v, d_o, l, delta, dk, dv, nullptr, (int)nh, (int)T, 0, BH,
                              rs(q_strides), rs(k_strides), rs(v_strides), rs(do_strides), sl,
                              sdk, sdv, scale, st);
  });
  return check_launch("flash_attention_bwd_dkdv");
}
}  // namespace

extern "C" int cta_flash_attention_bwd_dq(const float* q, const int64_t* q_strides,
                                          const float* k, const int64_t* k_strides,
                                          const float* v, const int64_t* v_strides,
                                          const float* d_o, const int64_t* do_strides,
                                          const float* l, const int64_t* l_strides,
                                          const float* delta, int64_t B, int64_t nh, int64_t T,
                                          int64_t hs, int causal, float* dq, void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (int rc = check_bwd_inputs(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l,
                                l_strides, delta))
    return rc;
  if (!dq || !aligned16(dq)) return fail(CTA_ERR_LAYOUT, "dQ must be a 16-byte aligned pointer");
  // (read only: without O the kernel reads delta)
  return bwd_dq_impl(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l, l_strides,
                     const_cast<float*>(delta), B, nh, T, hs, causal, dq, dense_out(nh, T, hs),
                     as_stream(stream));
}

extern "C" int cta_flash_attention_bwd_dq_delta(
    const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
    const float* v, const int64_t* v_strides, const float* o, const int64_t* o_strides,
    const float* d_o, const int64_t* do_strides, const float* l, const int64_t* l_strides,
    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal, float* delta, float* dq,
    void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (!attn_layout_ok(o, o_strides))
    return fail(CTA_ERR_LAYOUT,
                "flash_attention_bwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                "aligned O/dO");
  if (int rc = check_bwd_inputs(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l,
                                l_strides, delta))
    return rc;
  if (!dq || !aligned16(dq)) return fail(CTA_ERR_LAYOUT, "dQ must be a 16-byte aligned pointer");
  return bwd_dq_impl(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l, l_strides,
                     delta, B, nh, T, hs, causal, dq, dense_out(nh, T, hs), as_stream(stream), o,
                     rs(o_strides));
}

extern "C" int cta_flash_attention_bwd_dkdv(const float* q, const int64_t* q_strides,
                                            const float* k, const int64_t* k_strides,
                                            const float* v, const int64_t* v_strides,
                                            const float* d_o, const int64_t* do_strides,
                                            const float* l, const int64_t* l_strides,
                                            const float* delta, int64_t B, int64_t nh, int64_t T,
                                            int64_t hs, int causal, float* dk, float* dv,
                                            void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (int rc = check_bwd_inputs(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l,
                                l_strides, delta))
    return rc;
  if (!dk || !dv || !aligned16(dk) || !aligned16(dv))
    return fail(CTA_ERR_LAYOUT, "dK/dV must be 16-byte aligned pointers");
  const RowStrides dense = dense_out(nh, T, hs);
  return bwd_dkdv_impl(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l, l_strides,
                       delta, B, nh, T, hs, causal, dk, dense, dv, dense, as_stream(stream));
}

extern "C" int64_t cta_flash_attention_bwd_workspace(int64_t B, int64_t nh, int64_t T,
                                                     int64_t hs, int causal) {
  if (B <= 0 || nh <= 0 || T <= 0 || (hs != 32 && hs != 64 && hs != 128)) return 0;
  return B * nh * ds_tiles_per_head(T, causal != 0) * kDsTileFloats * (int64_t)sizeof(float);
}

extern "C" int64_t cta_flash_attention_bwd_split_workspace(int64_t B, int64_t nh, int64_t T,
                                                           int64_t hs, int causal) {
  if (B <= 0 || nh <= 0 || T <= 0 || (hs != 32 && hs != 64 && hs != 128) ||
      B * nh > ((int64_t)1 << 24) || T > ((int64_t)1 << 24))
    return 0;
  bool split = false;
  dispatch_hs_causal(hs, causal, [&]<int HS, bool C>() { split = dkdv_split<HS, C>((int)T, (int)(B * nh)); });
  return split ? 2 * B * nh * T * hs * (int64_t)sizeof(float) : 0;
}

extern "C" int cta_flash_attention_bwd_dkdv_store_ds(
    const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
    const float* v, const int64_t* v_strides, const float* d_o, const int64_t* do_strides,
    const float* l, const int64_t* l_strides, const float* delta, int64_t B, int64_t nh,
    int64_t T, int64_t hs, int causal, float* dk, float* dv, float* ds_workspace,
    void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (int rc = check_bwd_inputs(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l,
                                l_strides, delta))
    return rc;
  if (!dk || !dv || !aligned16(dk) || !aligned16(dv) || !ds_workspace || !aligned16(ds_workspace))
    return fail(CTA_ERR_LAYOUT, "dK/dV and the dS workspace must be 16-byte aligned pointers");
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const LStrides sl{l_strides[0], l_strides[1], l_strides[2]};
  hipStream_t st = as_stream(stream);
  dispatch_hs_causal(hs, causal, [&]<int HS, bool C>() {
    launch_dkdv<HS, C, true>(q, k, v, d_o, l, delta, dk, dv, ds_workspace, (int)nh, (int)T, 0,
                             (int)(B * nh), rs(q_strides), rs(k_strides), rs(v_strides),
                             rs(do_strides), sl, dense_out(nh, T, hs), dense_out(nh, T, hs),
                             scale, st);
  });
  return check_launch("flash_attention_bwd_dkdv_store_ds");
}

extern "C" int cta_flash_attention_bwd_dq_from_ds(const float* k, const int64_t* k_strides,
                                                  const float* ds_workspace, int64_t B,
                                                  int64_t nh, int64_t T, int64_t hs, int causal,
                                                  float* dq, void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (!attn_layout_ok(k, k_strides))
    return fail(CTA_ERR_LAYOUT,
                "flash_attention_bwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                "aligned K");
  if (!dq || !aligned16(dq) || !ds_workspace || !aligned16(ds_workspace))
    return fail(CTA_ERR_LAYOUT, "dQ and the dS workspace must be 16-byte aligned pointers");
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  hipStream_t st = as_stream(stream);
  dispatch_hs_causal(hs, causal, [&]<int HS, bool C>() {
    launch_dq_ds<HS, C>(k, ds_workspace, dq, (int)nh, (int)T, 0, (int)(B * nh), rs(k_strides),
                        dense_out(nh, T, hs), scale, st);
  });
  return check_launch("flash_attention_bwd_dq_from_ds");
}

extern "C" int cta_flash_attention_bwd_strided(
    const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
    const float* v, const int64_t* v_strides, const float* o, const int64_t* o_strides,
    const float* d_o, const int64_t* do_strides, const float* l, const int64_t* l_strides,
    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal, float* dq,
    const int64_t* dq_strides, float* dk, const int64_t* dk_strides, float* dv,
    const int64_t* dv_strides, float* delta, float* workspace, int64_t workspace_bytes,
    void* stream) {
  const int64_t head_bytes = cta_flash_attention_bwd_workspace(1, 1, T, hs, causal);
  const bool stored = workspace != nullptr && head_bytes != 0 && workspace_bytes >= head_bytes;
  if (stored) {
    if (int rc = cta_flash_attention_bwd_delta(o, o_strides, d_o, do_strides, B, nh, T, hs,
                                               delta, stream))
      return rc;
  } else {
    // the recompute schedule's dQ stage forms delta itself: the delta pass's checks only
    if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
    if (B * nh * T > 0 && (!attn_layout_ok(o, o_strides) || !attn_layout_ok(d_o, do_strides)))
      return fail(CTA_ERR_LAYOUT,
                  "flash_attention_bwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                  "aligned O/dO");
  }
  if (B * nh * T == 0) return CTA_OK;
  if (int rc = check_bwd_inputs(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l,
                                l_strides, delta))
    return rc;
  if (!attn_layout_ok(dq, dq_strides) || !attn_layout_ok(dk, dk_strides) ||
      !attn_layout_ok(dv, dv_strides))
    return fail(CTA_ERR_LAYOUT,
                "flash_attention_bwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                "aligned dQ/dK/dV");
  const RowStrides sdq = rs(dq_strides), sdk = rs(dk_strides), sdv = rs(dv_strides);
  hipStream_t st = as_stream(stream);
  if (!stored) {
    // The reference's schedule: dQ recomputes S and dP, and forms delta for dK/dV on the way
    // (no delta launch).
    if (int rc = bwd_dq_impl(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l,
                             l_strides, delta, B, nh, T, hs, causal, dq, sdq, st, o,
                             rs(o_strides)))
      return rc;
    return bwd_dkdv_impl(q, q_strides, k, k_strides, v, v_strides, d_o, do_strides, l,
                         l_strides, delta, B, nh, T, hs, causal, dk, sdk, dv, sdv, st);
  }
  if (!aligned16(workspace))
    return fail(CTA_ERR_LAYOUT, "the workspace must be a 16-byte aligned pointer");
  // Stored-dS schedule over chunks of equal head counts that fit the workspace.
  const int BH = (int)(B * nh);
  const int64_t fit = std::min<int64_t>(BH, workspace_bytes / head_bytes);
  const int64_t n_chunks = (BH + fit - 1) / fit;
  const int chunk = (int)((BH + n_chunks - 1) / n_chunks);
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const LStrides sl{l_strides[0], l_strides[1], l_strides[2]};
  // A small grid's dK/dV and dQ-from-dS stages split over twice the workgroups when the
  // workspace also holds the split's partial sums after every head's dS tiles (dK, dV; then,
  // once the dK/dV sum pass has read them, dQ in the same place).
  const int64_t ds_all = cta_flash_attention_bwd_workspace(B, nh, T, hs, causal);
  const int64_t split = cta_flash_attention_bwd_split_workspace(B, nh, T, hs, causal);
  float* part_ws = split > 0 && n_chunks == 1 && workspace_bytes >= ds_all + split
                       ? workspace + ds_all / (int64_t)sizeof(float)
                       : nullptr;
  for (int h0 = 0; h0 < BH; h0 += chunk) {
    const int n = std::min(chunk, BH - h0);
    dispatch_hs_causal(hs, causal, [&]<int HS, bool C>() {
      launch_dkdv<HS, C, true>(q, k, v, d_o, l, delta, dk, dv, workspace, (int)nh, (int)T, h0, n,
                               rs(q_strides), rs(k_strides), rs(v_strides), rs(do_strides), sl,
                               sdk, sdv, scale, st, nullptr, {}, part_ws);
      launch_dq_ds<HS, C>(k, workspace, dq, (int)nh, (int)T, h0, n, rs(k_strides), sdq, scale,
                          st, part_ws);
    });
    if (int rc = check_launch("flash_attention_bwd")) return rc;
  }
  return CTA_OK;
}

extern "C" int cta_flash_attention_bwd(const float* q, const int64_t* q_strides, const float* k,
                                       const int64_t* k_strides, const float* v,
                                       const int64_t* v_strides, const float* o,
                                       const int64_t* o_strides, const float* d_o,
                                       const int64_t* do_strides, const float* l,
                                       const int64_t* l_strides, int64_t B, int64_t nh,
                                       int64_t T, int64_t hs, int causal, float* dq, float* dk,
                                       float* dv, float* delta, float* workspace,
                                       int64_t workspace_bytes, void* stream) {
  const int64_t ds[4] = {nh * T * hs, T * hs, hs, 1};  // dense (B, nh, T, hs) outputs
  return cta_flash_attention_bwd_strided(q, q_strides, k, k_strides, v, v_strides, o, o_strides,
                                         d_o, do_strides, l, l_strides, B, nh, T, hs, causal, dq,
                                         ds, dk, ds, dv, ds, delta, workspace, workspace_bytes,
                                         stream);
}

extern "C" int cta_flash_attention_bwd_fold_delta(
    const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
    const float* v, const int64_t* v_strides, const float* o, const int64_t* o_strides,
    const float* d_o, const int64_t* do_strides, const float* l, const int64_t* l_strides,
    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal, float* dq, float* dk, float* dv,
    float* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (!attn_layout_ok(q, q_strides) || !attn_layout_ok(k, k_strides) ||
      !attn_layout_ok(v, v_strides) || !attn_layout_ok(o, o_strides) ||
      !attn_layout_ok(d_o, do_strides))
    return fail(CTA_ERR_LAYOUT,
                "flash_attention_bwd needs unit d-stride, strides divisible by 4, time strides below 2^23 and 16-byte "
                "aligned Q/K/V/O/dO");
  if (!l_ok(l, l_strides)) return fail(CTA_ERR_INVALID_ARGUMENT, "null L pointer");
  const int64_t head_bytes = cta_flash_attention_bwd_workspace(1, 1, T, hs, causal);
  if (workspace == nullptr || workspace_bytes < head_bytes)
    return fail(CTA_ERR_INVALID_ARGUMENT,
                "flash_attention_bwd_fold_delta needs a dS workspace of at least one head (" +
                    std::to_string(head_bytes) + " bytes)");
  if (!dq || !dk || !dv || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) ||
      !aligned16(workspace))
    return fail(CTA_ERR_LAYOUT, "dQ/dK/dV and the workspace must be 16-byte aligned pointers");
  const int BH = (int)(B * nh);
  const int64_t fit = std::min<int64_t>(BH, workspace_bytes / head_bytes);
  const int64_t n_chunks = (BH + fit - 1) / fit;
  const int chunk = (int)((BH + n_chunks - 1) / n_chunks);
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const LStrides sl{l_strides[0], l_strides[1], l_strides[2]};
  hipStream_t st = as_stream(stream);
  for (int h0 = 0; h0 < BH; h0 += chunk) {
    const int n = std::min(chunk, BH - h0);
    dispatch_hs_causal(hs, causal, [&]<int HS, bool C>() {
      launch_dkdv<HS, C, true, true>(q, k, v, d_o, l, nullptr, dk, dv, workspace, (int)nh,
                                     (int)T, h0, n, rs(q_strides), rs(k_strides), rs(v_strides),
                                     rs(do_strides), sl, dense_out(nh, T, hs),
                                     dense_out(nh, T, hs), scale, st, o, rs(o_strides));
      launch_dq_ds<HS, C>(k, workspace, dq, (int)nh, (int)T, h0, n, rs(k_strides),
                          dense_out(nh, T, hs), scale, st);
    });
    if (int rc = check_launch("flash_attention_bwd_fold_delta")) return rc;
  }
  return CTA_OK;
}
