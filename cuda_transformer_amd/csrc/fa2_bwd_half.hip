// FlashAttention-2 backward with 16-bit (BF16 or FP16) Q, K, V, O, dO (FP32 L), FP32
// accumulation, CDNA4 MFMA (v_mfma_f32_32x32x16_bf16 / _f16).  dQ, dK, dV are written in the
// input type.  Written for BF16; the FP16 instance differs only in the element type and the
// MFMA (Half16<E>), and stores dS in FP16.
//
// The semantics are those of the FP32 backward (Transformer_kernels/flash_attention.cuh:175-504):
//   delta_i = sum_d O_id dO_id,  P_ij = e^{S_ij - L_i},  dP_ij = dO_i . v_j,
//   dS_ij = P_ij (dP_ij - delta_i),  dV_j = sum_i P_ij dO_i,  dK_j = s sum_i dS_ij q_i,
//   dQ_i = s sum_j dS_ij k_j,  S = s q.k, s = 1/sqrt(hs), causal mask j > i.
// S, dP, delta and dS are FP32; P and dS are rounded to BF16 as MFMA operands, and dS is stored
// in BF16 for the dQ stage.  Two schedules, as in FP32, both atomics-free and deterministic:
//  * stored dS (given a workspace of at least one head's tiles): delta, then a dK/dV stage that
//    also writes every dS tile, then dQ = s dS K from the stored tiles;
//  * recompute (no workspace; the reference's schedule): a dQ stage that recomputes S and dP
//    from L and forms delta itself (the delta pass's sums, the same bits), then dK/dV without
//    the store.  dK and dV are bitwise those of the stored schedule (the same kernel body); dQ
//    differs by the rounding of its sums.
//
// gfx950 layout (the 16-bit forward's trick, see fa2_fwd_half.hip):
//  * dK/dV: a wave owns 32 key rows and keeps k, v of its key row in registers as the B
//    operands of S = Q K^T and dP = dO V^T, read row-wise from [query][d] images of the Q and
//    dO tiles.  S and dP then hold one key per lane; P and dS, rounded to BF16, are the B
//    operands of dV^T += dO^T P and dK^T += Q^T dS, whose A operands come from transposed
//    [d][query] images with bits 2 and 3 of the query index swapped (kt_pos).  Each stage's
//    Q / dO tile therefore goes to LDS twice, row-wise and transposed.
//  * dS tiles go through a per-wave LDS transpose and out to HBM in the dQ stage's operand
//    order: in tile (ib, jb), lane l = 32 h + c of step s reads 8 consecutive keys
//    16 s + 8 h .. +7 of query c at offset 8 (32 (2 s + h) + c), one 16-byte load.
//  * dQ: a wave owns 32 query rows; K tiles go to LDS transposed ([d][key]) and the stored dS
//    tiles straight into registers as the B operand of dQ^T += K^T dS^T.
#include "cta_common.hpp"

namespace cta {
namespace {

struct RowStridesH {
  int64_t b, h, t;  // element strides of the batch, head and time axes (d-stride is 1)
};

constexpr int kDsTileHalf = 1024;  // 16-bit elements of one stored 32x32 dS tile

// ------------------------------------------------------------------------------------
// delta = rowsum(O * dO), FP32 from BF16 rows; G = hs/8 lanes per row, 16 bytes each.
template <class E, int HS>
__global__ __launch_bounds__(256) void fa2_bwd_delta_half_kernel(const E* __restrict__ O,
                                                                 const E* __restrict__ dO,
                                                                 float* __restrict__ delta,
                                                                 int nh, int T, int64_t rows,
                                                                 RowStridesH so,
                                                                 RowStridesH sdo) {
  constexpr int G = HS / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / G;
  const int c8 = (int)(gid % G);
  float acc = 0.0f;
  if (row < rows) {
    const int64_t bh = row / T;
    const int t = (int)(row - bh * T);
    const int64_t b = bh / nh, h = bh - b * nh;
    const vec8_t<E> o = ld8<E>(O + b * so.b + h * so.h + (int64_t)t * so.t + 8 * c8);
    const vec8_t<E> g = ld8<E>(dO + b * sdo.b + h * sdo.h + (int64_t)t * sdo.t + 8 * c8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf((float)o[e], (float)g[e], acc);
  }
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (row < rows && c8 == 0) delta[row] = acc;
}

// ------------------------------------------------------------------------------------
// dK, dV and the stored dS tiles.  Workgroup = WAVES x 32 key rows; query stages of BN rows
// (BN / 32 sub-tiles of 32, taken in the stage walk's direction), global -> registers -> LDS,
// double buffered, one barrier per stage.  Heads [bh_base, bh_base + BH); the dS tiles go to
// dsw, heads indexed from bh_base.  MINW: waves per SIMD the register budget is held to.
// hs = 32 and 64: eight waves (256 key rows) share each 64-row query stage, one workgroup per
// CU (115 KB of LDS at hs = 64), two waves per SIMD.  A stage then holds 1024 cycles of MFMA
// work per wave instead of 512, which hides the latency of the next stage's loads (the 4-wave,
// 32-row kernel waited on them: 57% of its wave-cycles were dependency waits), and every
// staged Q / dO row serves twice the keys.  Measured against four waves and 32-row stages
// (bitwise-identical gradients at T = 4096): causal backward 1.56-1.58 vs 1.70-1.71 ms, non-
// causal equal at config 2 and 4.5% faster at B1 H16 N8192.  Eight waves with 32-row stages
// were 10% slower.  hs = 128 keeps four waves, one per SIMD.
template <int HS, bool CAUSAL>
struct DkdvHalfCfg {
  static constexpr int WAVES = HS == 128 ? 4 : 8, BN = HS == 128 ? 32 : 64;
  static constexpr int MINW = HS == 128 ? 1 : 2;
};

template <class E, int HS, bool CAUSAL, int WAVES, int BN, int MINW, bool STORE>
__global__ __launch_bounds__(64 * WAVES, MINW) void fa2_bwd_dkdv_half_kernel(
    const E* __restrict__ Q, const E* __restrict__ K, const E* __restrict__ V,
    const E* __restrict__ dO, const float* __restrict__ Lg, const float* __restrict__ delta,
    E* __restrict__ dK, E* __restrict__ dV, E* __restrict__ dsw, int nh, int T,
    int bh_base, int BH, int n_ktiles, RowStridesH sq, RowStridesH sk, RowStridesH sv,
    RowStridesH sdo, RowStridesH sl, float scale, float scale_log2) {
  constexpr int THREADS = 64 * WAVES;
  constexpr int NSUB = BN / 32;      // 32-row sub-tiles per query stage
  constexpr int BM = 32 * WAVES;     // key rows per workgroup
  constexpr int RP = HS + 8;         // 16-bit pitch of a row image: conflict-free 16-byte reads
  constexpr int TP = BN + 8;         // 16-bit pitch of a transposed image row (one d)
  constexpr int XP = 32 + 8;         // 16-bit pitch of the dS transpose
  constexpr int CH = HS / 8;         // 16-byte chunks per row
  constexpr int PAIRS = BN / 2 * CH; // row-pair load tasks per tensor and stage
  constexpr int LOADS = (2 * PAIRS + THREADS - 1) / THREADS;  // load tasks per thread
  constexpr int QS = HS / 16;        // MFMA steps over d
  // Stage image, in bytes: Q rows, dO rows, Q^T, dO^T, L log2(e), -delta.
  constexpr int B_ROWS = BN * RP * 2, B_TRS = HS * TP * 2;
  constexpr int OFF_GR = B_ROWS, OFF_QT = 2 * B_ROWS, OFF_GT = 2 * B_ROWS + B_TRS;
  constexpr int OFF_L = 2 * B_ROWS + 2 * B_TRS, OFF_D = OFF_L + BN * 4;
  constexpr int STAGE = OFF_D + BN * 4;
  // per wave: one dS transpose buffer per sub-tile (none without the dS store)
  constexpr int XPOSE = STORE ? NSUB * 32 * XP * 2 : 0;
  static_assert(STAGE % 16 == 0 && OFF_QT % 16 == 0 && OFF_L % 16 == 0, "16-byte aligned images");
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * STAGE + WAVES * XPOSE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  const int per_head = CAUSAL ? (n_ktiles + 1) / 2 : n_ktiles;
  const int w = xcd_work_item(blockIdx.x, BH * per_head);
  if (w >= BH * per_head) return;
  const int bh_local = w / per_head;
  const int p = w - bh_local * per_head;
  const int bh = bh_base + bh_local;
  const int b = bh / nh, h = bh - b * nh;

  const E* Qb = Q + b * sq.b + h * sq.h;
  const E* dOb = dO + b * sdo.b + h * sdo.h;
  const float* Lb = Lg + b * sl.b + h * sl.h;
  const float* Db = delta + (int64_t)bh * T;
  const int nb = (T + 31) / 32;
  E* xw = reinterpret_cast<E*>(smem + 2 * STAGE + wave * XPOSE);
  E* dsh = STORE ? dsw + (int64_t)bh_local * ds_tiles_per_head(T, CAUSAL) * kDsTileHalf : nullptr;

  const int n_pass = (CAUSAL && n_ktiles - 1 - p != p) ? 2 : 1;
  for (int pass = 0; pass < n_pass; ++pass) {
  const int kt = CAUSAL ? (pass == 0 ? p : n_ktiles - 1 - p) : p;
  const int j0 = kt * BM + wave * 32;  // first key row of this wave
  const int my_j = j0 + col;

  // k and v of this lane's key row, d = 16 s + 8 half + 0..7 for step s.
  vec8_t<E> kf[QS], vf[QS];
  if (my_j < T) {
    const E* kp = K + b * sk.b + h * sk.h + (int64_t)my_j * sk.t + 8 * half;
    const E* vp = V + b * sv.b + h * sv.h + (int64_t)my_j * sv.t + 8 * half;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      kf[s] = ld8<E>(kp + 16 * s);
      vf[s] = ld8<E>(vp + 16 * s);
    }
  } else {
#pragma unroll
    for (int s = 0; s < QS; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) { kf[s][j] = (E)0.0f; vf[s][j] = (E)0.0f; }
  }

  // The k and v rows are complete before the stage loop on every path into it.  Otherwise the
  // compiler, which cannot prove that, waits for them inside each stage, and since the
  // counter is in order that wait also drains the next stage's loads issued just before.
  vm_wait_all();

  f32x16 dkacc[HS / 32], dvacc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) { dkacc[d] = zero16(); dvacc[d] = zero16(); }

  const int q_begin = CAUSAL ? (kt * BM / BN) : 0;  // first query stage that can see these keys
  const int n_stages = (T + BN - 1) / BN;
  const bool wave_stores = STORE && j0 < T;

  // Register-staged loads of one query stage: Q and dO rows, L log2(e) and -delta.
  // A load task is rows 2 rp and 2 rp + 1 of one 16-byte chunk ch of Q or of dO; it goes to LDS
  // row-wise and transposed, the two rows' values for one d as one 32-bit store (kt_pos keeps
  // rows 2 rp and 2 rp + 1 adjacent).  Tasks [0, BN/2 * CH) are Q, the rest dO; PAIRS is a
  // multiple of 64, so the tensor is the same for a whole wave.
  // Rows past T (ragged last stage) are read clamped to row T - 1: their L and -delta are 0 and
  // the mask sets their P to 0, so dS = 0 there and they add nothing to dK, dV or dQ.
  // With fewer tasks than threads the first waves take them (wave-uniform).
  static_assert(PAIRS % 64 == 0, "load tensor must be wave-uniform");
  auto task_live = [&](int u) {
    return 2 * PAIRS % THREADS == 0 || tid + THREADS * u < 2 * PAIRS;
  };
  uint4 st2[LOADS][2];
  float lst = 0.0f, dst = 0.0f;  // L and delta of one query row
  // BN / 2 consecutive lanes take the row pairs of one chunk, so a transposed store
  // instruction spreads over the pair positions of one or two chunks.
  auto task_of = [&](int u, int& tensor, int& rp, int& ch) {
    const int c = tid + THREADS * u;
    tensor = __builtin_amdgcn_readfirstlane(c / PAIRS);
    const int rem = c - tensor * PAIRS;
    rp = rem % (BN / 2);
    ch = rem / (BN / 2);
  };
  const E* tbase[LOADS];
  int64_t tstride[LOADS], toff[LOADS][2];
#pragma unroll
  for (int u = 0; u < LOADS; ++u) {
    int tensor, rp, ch;
    task_of(u, tensor, rp, ch);
    tbase[u] = tensor == 0 ? Qb : dOb;  // (unused for a dead task)
    tstride[u] = tensor == 0 ? sq.t : sdo.t;
#pragma unroll
    for (int e = 0; e < 2; ++e) toff[u][e] = (int64_t)(2 * rp + e) * tstride[u] + 8 * ch;
  }
  auto gload = [&](int stage) {
    const int r0 = stage * BN;
    if (r0 + BN <= T) {
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        if (!task_live(u)) continue;
        const E* sb = tbase[u] + (int64_t)r0 * tstride[u];
#pragma unroll
        for (int e = 0; e < 2; ++e) st2[u][e] = *reinterpret_cast<const uint4*>(sb + toff[u][e]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        if (!task_live(u)) continue;
        int tensor, rp, ch;
        task_of(u, tensor, rp, ch);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int i = min(r0 + 2 * rp + e, T - 1);
          st2[u][e] = *reinterpret_cast<const uint4*>(tbase[u] + (int64_t)i * tstride[u] + 8 * ch);
        }
      }
    }
    if (tid < BN) {
      const int i = r0 + tid;
      lst = i < T ? Lb[(int64_t)i * sl.t] : 0.0f;
      dst = i < T ? Db[i] : 0.0f;
    }
  };
  auto lstore = [&](int buf) {
    unsigned char* base = smem + buf * STAGE;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      if (!task_live(u)) continue;
      int tensor, rp, ch;
      task_of(u, tensor, rp, ch);
      E* rows = reinterpret_cast<E*>(base + (tensor == 0 ? 0 : OFF_GR));
      E* trs = reinterpret_cast<E*>(base + (tensor == 0 ? OFF_QT : OFF_GT));
      *reinterpret_cast<uint4*>(rows + (2 * rp) * RP + 8 * ch) = st2[u][0];
      *reinterpret_cast<uint4*>(rows + (2 * rp + 1) * RP + 8 * ch) = st2[u][1];
      const uint32_t* e0 = reinterpret_cast<const uint32_t*>(&st2[u][0]);
      const uint32_t* e1 = reinterpret_cast<const uint32_t*>(&st2[u][1]);
      uint32_t* col2 = reinterpret_cast<uint32_t*>(trs + kt_pos(2 * rp));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        col2[(8 * ch + 2 * t) * (TP / 2)] = pack_lo16(e0[t], e1[t]);
        col2[(8 * ch + 2 * t + 1) * (TP / 2)] = pack_hi16(e0[t], e1[t]);
      }
    }
    if (tid < BN) {
      // Scaled here, not at the load, where the arithmetic would wait for the loads to land.
      reinterpret_cast<float*>(base + OFF_L)[tid] = lst * kLog2e;
      reinterpret_cast<float*>(base + OFF_D)[tid] = -dst;
    }
  };

  // Tiles whose every query row precedes every key row are skipped (dS = 0, nothing stored).
  auto live = [&](int ii0) { return ii0 < T && !(CAUSAL && ii0 + 31 < j0); };
  // The dS tiles of query stage `stage`, from the transpose buffers to the workspace.
  auto flush = [&](int stage) {
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int ii0 = stage * BN + sub * 32;
      if (!live(ii0)) continue;
      E* gtile = dsh + ds_tile_index(ii0 / 32, j0 / 32, nb, CAUSAL) * kDsTileHalf;
      const E* xs = xw + sub * 32 * XP;
      wave_lds_fence();
#pragma unroll
      for (int s = 0; s < 2; ++s)
        st8_stream<E>(gtile + 8 * (32 * (2 * s + half) + col), ld8<E>(xs + col * XP + 16 * s + 8 * half));
      wave_lds_fence();
    }
  };

  // Stage order: with a causal mask the first (long) pass walks its query stages downward and
  // the second (short) pass upward, so a head's workgroups share each streamed stage in L2.
  const int n_steps = n_stages - q_begin;
  const bool down = CAUSAL && pass == 0;
  auto stage_at = [&](int i) { return down ? n_stages - 1 - i : q_begin + i; };
  if (n_steps > 0) {
    gload(stage_at(0));
    lstore(0);
  }
  __syncthreads();

  for (int i = 0; i < n_steps; ++i) {
    const int s_idx = stage_at(i);
    const int buf = i & 1;
    if (i + 1 < n_steps) gload(stage_at(i + 1));
    if (wave_stores && i > 0) flush(stage_at(i - 1));
    const unsigned char* base = smem + buf * STAGE;
    const E* qr = reinterpret_cast<const E*>(base);
    const E* gr = reinterpret_cast<const E*>(base + OFF_GR);
    const E* qt = reinterpret_cast<const E*>(base + OFF_QT);
    const E* gt = reinterpret_cast<const E*>(base + OFF_GT);
    const float* ls = reinterpret_cast<const float*>(base + OFF_L);
    const float* ds = reinterpret_cast<const float*>(base + OFF_D);
    // hs 128 (one wave per SIMD, nothing to hide the LDS latency behind): the A operands of
    // dV^T += dO^T P and dK^T += Q^T dS are read before the S and dP MFMAs, so they are in
    // registers when the exponentials finish.  A/B in one process, bitwise-equal gradients:
    // stored-dS backward +2.3% at B4 H32 N4096 hs 128; no change at hs 32 / 64 (two waves per
    // SIMD), which keep the reads beside their MFMAs.
    constexpr bool PRE = HS == 128;
    typedef vec8_t<E> AOps[HS / 32][2];
    // S = Q K^T and dP = dO V^T of sub-tile `sub`: lane holds column my_j, rows
    // ii0 + R(r, half).  The stage holds -delta, and the dP products accumulate onto it:
    // pacc = dP - delta.
    auto score = [&](int sub, f32x16& sacc, f32x16& pacc, AOps& gop, AOps& qop) {
      sacc = zero16();
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 dv = ld4(ds + sub * 32 + 8 * g + 4 * half);
        pacc[4 * g + 0] = dv.x;
        pacc[4 * g + 1] = dv.y;
        pacc[4 * g + 2] = dv.z;
        pacc[4 * g + 3] = dv.w;
      }
      if constexpr (PRE) {
#pragma unroll
        for (int d = 0; d < HS / 32; ++d)
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            gop[d][s] = ld8<E>(gt + (d * 32 + col) * TP + sub * 32 + 16 * s + 8 * half);
            qop[d][s] = ld8<E>(qt + (d * 32 + col) * TP + sub * 32 + 16 * s + 8 * half);
          }
      }
#pragma unroll
      for (int s = 0; s < QS; ++s)
        sacc = Half16<E>::mfma(ld8<E>(qr + (sub * 32 + col) * RP + 16 * s + 8 * half), kf[s], sacc);
#pragma unroll
      for (int s = 0; s < QS; ++s)
        pacc = Half16<E>::mfma(ld8<E>(gr + (sub * 32 + col) * RP + 16 * s + 8 * half), vf[s], pacc);
      if constexpr (PRE) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * QS + 4 * (HS / 32), 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * QS, 0);
      }
    };
    // P, dV, dS and dK of sub-tile `sub` (query rows ii0..) from its S and dP - delta.
    auto finish = [&](int sub, int ii0, f32x16& sacc, const f32x16& pacc, const AOps& gop,
                      const AOps& qop) {
      // P = e^{S - L}; masked entries (and, for the stored dS, key rows past T) are exactly 0.
      // The stage holds L log2(e).  Two explicit paths: left to the compiler, the masked form
      // is if-converted into per-element selects that every tile then pays for.
      auto exp_scores = [&]<bool MASKED>() {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 lv = ld4(ls + sub * 32 + 8 * g + 4 * half);
          const float lr[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            float x = fmaf(sacc[r], scale_log2, -lr[e]);
            if (MASKED) {
              const int qi = ii0 + 8 * g + 4 * half + e;
              if ((CAUSAL && my_j > qi) || qi >= T || my_j >= T) x = -INFINITY;  // 2^x = 0
            }
            sacc[r] = fast_exp2(x);
          }
        }
      };
      if ((CAUSAL && ii0 < j0 + 31) || (ii0 + 32 > T) || (j0 + 32 > T))
        exp_scores.template operator()<true>();
      else
        exp_scores.template operator()<false>();
      vec8_t<E> pb[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) pb[r >> 3][r & 7] = (E)sacc[r];

      // dV^T += dO^T P
#pragma unroll
      for (int d = 0; d < HS / 32; ++d)
#pragma unroll
        for (int s = 0; s < 2; ++s)
          dvacc[d] = Half16<E>::mfma(
              PRE ? gop[d][s] : ld8<E>(gt + (d * 32 + col) * TP + sub * 32 + 16 * s + 8 * half),
              pb[s], dvacc[d]);

      // dS = P (dP - delta)
      vec8_t<E> db[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) db[r >> 3][r & 7] = (E)(sacc[r] * pacc[r]);

      // dS tile into the transpose buffer as [query][key]: lane (col, half) holds
      // dS[ii0 + R(r, half)][j0 + col].  A wave's LDS operations complete in order, so no
      // barrier separates the write, the read in flush() and the next write.
      // Each converted pair is stored as its low and its high half (ds_write_b16 and
      // ds_write_b16_d16_hi), without unpacking it.
      if constexpr (STORE) {
        uint16_t* xw16 = reinterpret_cast<uint16_t*>(xw + sub * 32 * XP);
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          uint32_t pk = reinterpret_cast<const uint32_t*>(&db[r >> 3])[(r & 7) >> 1];
          // Opaque to the optimiser, which would otherwise convert each half again on its own.
          asm("" : "+v"(pk));
          xw16[mfma_row(r, half) * XP + col] = (uint16_t)pk;
          xw16[mfma_row(r + 1, half) * XP + col] = (uint16_t)(pk >> 16);
        }
      }

      // dK^T += Q^T dS
#pragma unroll
      for (int d = 0; d < HS / 32; ++d)
#pragma unroll
        for (int s = 0; s < 2; ++s)
          dkacc[d] = Half16<E>::mfma(
              PRE ? qop[d][s] : ld8<E>(qt + (d * 32 + col) * TP + sub * 32 + 16 * s + 8 * half),
              db[s], dkacc[d]);
    };

    // Sub-tiles in the stage walk's direction, so a wave's dK / dV sums run over 32-row tiles
    // in the same order whatever the stage height.
#pragma unroll
    for (int k = 0; k < NSUB; ++k) {
      const int sub = down ? NSUB - 1 - k : k;
      const int ii0 = s_idx * BN + sub * 32;
      if (live(ii0)) {
        f32x16 sacc, pacc;
        AOps gop, qop;
        score(sub, sacc, pacc, gop, qop);
        finish(sub, ii0, sacc, pacc, gop, qop);
      }
    }  // sub-tiles
    if (i + 1 < n_steps) lstore(buf ^ 1);
    __syncthreads();
  }
  if (wave_stores && n_steps > 0) flush(stage_at(n_steps - 1));

  if (my_j < T) {
    E* kp = dK + ((int64_t)bh * T + my_j) * HS;
    E* vp = dV + ((int64_t)bh * T + my_j) * HS;
#pragma unroll
    for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        E k4[4], v4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          k4[e] = (E)(dkacc[d][4 * g + e] * scale);
          v4[e] = (E)dvacc[d][4 * g + e];
        }
        const int dc = d * 32 + 8 * g + 4 * half;
        *reinterpret_cast<uint2*>(kp + dc) = *reinterpret_cast<const uint2*>(k4);
        *reinterpret_cast<uint2*>(vp + dc) = *reinterpret_cast<const uint2*>(v4);
      }
    }
  }
  }  // pass: the stage loop ended on a barrier, so the next pass may refill LDS
}

// ------------------------------------------------------------------------------------
// dQ from the stored BF16 dS tiles: dQ^T += K^T dS^T.  Workgroup = 128 query rows (4 waves x
// 32); key stages of 64 rows go to LDS transposed ([d][key]); each wave loads its own dS tiles
// from the workspace straight into registers, one stage ahead.
template <class E, int HS, bool CAUSAL>
__global__ __launch_bounds__(256, HS == 128 ? 1 : 2) void fa2_bwd_dq_ds_half_kernel(
    const E* __restrict__ K, const E* __restrict__ dsw, E* __restrict__ dQ,
    int nh, int T, int bh_base, int BH, int n_qtiles, RowStridesH sk, float scale,
    int heads_per_xcd = 0) {
  constexpr int BN = 64;
  constexpr int NSUB = BN / 32;
  constexpr int BM = 128;
  constexpr int KTP = BN + 8;  // 16-bit pitch of a K^T row (one d, every key of the stage)
  constexpr int TILE = HS * KTP;
  constexpr int CH = HS / 8;
  __shared__ __attribute__((aligned(16))) E smem[2 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  // query-tile pairs (n-1-p, p), or (heads_per_xcd > 0) single tiles longest first (lpt_tile)
  int bh_local, qa, qb = -1;
  if (CAUSAL && heads_per_xcd > 0) {
    int rank;
    lpt_tile(blockIdx.x, heads_per_xcd, bh_local, rank);
    qa = n_qtiles - 1 - rank;
  } else {
    const int per_head = CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles;
    const int w = xcd_work_item(blockIdx.x, BH * per_head);
    if (w >= BH * per_head) return;
    bh_local = w / per_head;
    const int p = w - bh_local * per_head;
    qa = CAUSAL ? n_qtiles - 1 - p : p;
    if (CAUSAL && n_qtiles - 1 - p != p) qb = p;
  }
  const int bh = bh_base + bh_local;
  const int b = bh / nh, h = bh - b * nh;
  const E* Kb = K + b * sk.b + h * sk.h;
  const int nb = (T + 31) / 32;
  const E* dsh = dsw + (int64_t)bh_local * ds_tiles_per_head(T, CAUSAL) * kDsTileHalf;

  const int n_pass = qb >= 0 ? 2 : 1;
  for (int pass = 0; pass < n_pass; ++pass) {
  const int qt = pass == 0 ? qa : qb;
  const int i0 = qt * BM + wave * 32;
  const int my_i = i0 + col;
  const int ib = i0 / 32;

  f32x16 acc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) acc[d] = zero16();

  const int kv_end = CAUSAL ? min(T, (qt + 1) * BM) : T;
  const int n_stages = (kv_end + BN - 1) / BN;

  // Branch-free clamped loads: every stage issues the same loads, so the compiler counts them
  // exactly and a stage's MFMAs wait only for that stage's dS.  A thread loads rows 2 rp and
  // 2 rp + 1 of chunk ch and stores each d's pair as one 32-bit word of the K^T image.
  constexpr int KPAIRS = 32 * CH;              // K row-pair tasks per stage
  constexpr int KL = (KPAIRS + 255) / 256;     // ... per thread (hs = 32: waves 0 and 1 only)
  uint4 kst[2 * KL];
  // A wave's 64 tasks are 32 row pairs x 2 chunks: each transposed store instruction hits 64
  // distinct banks (the 32 pair positions, and the two chunks' d rows 32 banks apart).
  static_assert(BN == 64, "32 row pairs per stage");
  auto pair_of = [&](int u2, int& rp, int& ch) {
    rp = lane & 31;
    ch = 2 * (wave + 4 * u2) + (lane >> 5);
    return KPAIRS % 256 == 0 || ch < CH;
  };
  // K rows through a buffer resource over the stage's valid rows: keys past T read as zero, as
  // they must, since they meet finite dS columns.
  auto gload = [&](int stage) {
    const int j0 = stage * BN;
    const __amdgpu_buffer_rsrc_t rk =
        rows_rsrc16(Kb + (int64_t)j0 * sk.t, min(BN, T - j0), sk.t, HS);
#pragma unroll
    for (int u2 = 0; u2 < KL; ++u2) {
      int rp, ch;
      if (!pair_of(u2, rp, ch)) continue;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const u32x4 w = ld16_buffer(rk, ((2 * rp + e) * (int)sk.t + 8 * ch) * 2);
        kst[2 * u2 + e] = make_uint4(w.x, w.y, w.z, w.w);
      }
    }
  };
  auto lstore = [&](int buf) {
    E* kt = smem + buf * TILE;
#pragma unroll
    for (int u2 = 0; u2 < KL; ++u2) {
      int rp, ch;
      if (!pair_of(u2, rp, ch)) continue;
      const uint32_t* e0 = reinterpret_cast<const uint32_t*>(&kst[2 * u2]);
      const uint32_t* e1 = reinterpret_cast<const uint32_t*>(&kst[2 * u2 + 1]);
      uint32_t* col2 = reinterpret_cast<uint32_t*>(kt + 2 * rp);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        col2[(8 * ch + 2 * t) * (KTP / 2)] = pack_lo16(e0[t], e1[t]);
        col2[(8 * ch + 2 * t + 1) * (KTP / 2)] = pack_hi16(e0[t], e1[t]);
      }
    }
  };
  auto has_tile = [&](int jb) { return ib < nb && jb < nb && (!CAUSAL || jb <= ib); };
  const int ibc = min(ib, nb - 1);
  auto dsload = [&](int stage, vec8_t<E> (&dr)[NSUB][2]) {
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int jbc = min(stage * NSUB + sub, CAUSAL ? ibc : nb - 1);
      const E* src = dsh + ds_tile_index(ibc, jbc, nb, CAUSAL) * kDsTileHalf;
#pragma unroll
      for (int s = 0; s < 2; ++s) dr[sub][s] = ld8_stream<E>(src + 8 * (32 * (2 * s + half) + col));
    }
  };
  auto compute = [&](int stage, const E* kt, const vec8_t<E> (&dr)[NSUB][2]) {
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      if (!has_tile(stage * NSUB + sub)) continue;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int d = 0; d < HS / 32; ++d)
          acc[d] = Half16<E>::mfma(ld8<E>(kt + (d * 32 + col) * KTP + sub * 32 + 16 * s + 8 * half),
                             dr[sub][s], acc[d]);
    }
  };
  auto step = [&](int s, const vec8_t<E> (&cur)[NSUB][2], vec8_t<E> (&nxt)[NSUB][2]) {
    const int buf = s & 1;
    gload(s + 1);
    dsload(s + 1, nxt);
    compute(s, smem + buf * TILE, cur);
    lstore(buf ^ 1);
    __syncthreads();
  };

  vec8_t<E> dA[NSUB][2], dB[NSUB][2];
  dsload(0, dA);
  gload(0);
  lstore(0);
  __syncthreads();
  const int n_stages2 = (n_stages + 1) & ~1;
  for (int s = 0; s < n_stages2; s += 2) {
    step(s, dA, dB);
    step(s + 1, dB, dA);
  }

  if (my_i < T) {
    E* op = dQ + ((int64_t)bh * T + my_i) * HS;
#pragma unroll
    for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        E q4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) q4[e] = (E)(acc[d][4 * g + e] * scale);
        *reinterpret_cast<uint2*>(op + d * 32 + 8 * g + 4 * half) =
            *reinterpret_cast<const uint2*>(q4);
      }
    }
  }
  }  // pass: the stage loop ended on a barrier, so the next pass may refill LDS
}

// ------------------------------------------------------------------------------------
// dQ without a workspace: the reference's dQ stage (flash_attention.cuh:216-354), which
// recomputes S and dP from L and delta instead of reading stored dS tiles.  The 16-bit
// forward's skeleton: workgroup = 128 query rows (4 waves x 32), key stages of 64 rows,
// global -> registers -> LDS, double buffered, one barrier per stage; causal workgroups take
// query-tile pairs and the second pass walks its stages downward.  A lane keeps its query
// row's q and dO (the B operands of S^T = K Q^T and dP^T = V dO^T), L log2(e) and delta.  Each
// stage goes to LDS as K rows (S), V rows (dP) and K^T with kt_pos (the A operand of
// dQ^T += K^T dS^T, whose B operand is the lane's dS^T registers, as P^T is in the forward).
// It also forms delta = rowsum(O dO) from its rows (the sums of fa2_bwd_delta_half_kernel in
// the same order, so the same bits) and writes it for the dK/dV stage that runs after it:
// the recompute schedule needs no delta launch.
template <class E, int HS, bool CAUSAL>
__global__ __launch_bounds__(256, HS == 128 ? 1 : 2) void fa2_bwd_dq_half_kernel(
    const E* __restrict__ Q, const E* __restrict__ K, const E* __restrict__ V,
    const E* __restrict__ dO, const E* __restrict__ Og, const float* __restrict__ Lg,
    float* __restrict__ delta, E* __restrict__ dQ, int nh, int T, int BH, int n_qtiles,
    RowStridesH sq, RowStridesH sk, RowStridesH sv, RowStridesH sdo, RowStridesH so,
    RowStridesH sl, float scale, float scale_log2, int heads_per_xcd = 0) {
  constexpr int BN = 64;             // keys per stage
  constexpr int NSUB = BN / 32;
  constexpr int BM = 128;
  constexpr int RP = HS + 8;         // 16-bit pitch of a K / V row image
  constexpr int TP = BN + 8;         // 16-bit pitch of a K^T row (one d, every key of the stage)
  constexpr int RTILE = BN * RP, TTILE = HS * TP;
  constexpr int STAGE = 2 * RTILE + TTILE;  // K rows, V rows, K^T
  constexpr int CH = HS / 8;         // 16-byte chunks per row
  constexpr int QS = HS / 16;        // MFMA steps over d
  constexpr int KPAIRS = 32 * CH;    // K row-pair tasks per stage
  constexpr int KL = (KPAIRS + 255) / 256;
  constexpr int VLOADS = BN * CH / 256;
  static_assert(BN * CH % 256 == 0 && BN == 64, "stage must split evenly over 256 threads");
  __shared__ __attribute__((aligned(16))) E smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  // query-tile pairs (n-1-p, p), or (heads_per_xcd > 0) single tiles longest first (lpt_tile)
  int bh, qa, qb = -1;
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
  const E* Kb = K + b * sk.b + h * sk.h;
  const E* Vb = V + b * sv.b + h * sv.h;

  const int n_pass = qb >= 0 ? 2 : 1;
  for (int pass = 0; pass < n_pass; ++pass) {
  const int qt = pass == 0 ? qa : qb;
  const int i0 = qt * BM + wave * 32;
  const int my_i = i0 + col;

  // This lane's query row: q and dO at d = 16 s + 8 half + 0..7 for step s, L log2(e), delta.
  // Rows past T hold zeros: dO = 0 and delta = 0 make their dS 0, and their dQ is not stored.
  vec8_t<E> qf[QS], gf[QS];
  float lrow = 0.0f, drow = 0.0f;
  if (my_i < T) {
    const E* qp = Q + b * sq.b + h * sq.h + (int64_t)my_i * sq.t + 8 * half;
    const E* gp = dO + b * sdo.b + h * sdo.h + (int64_t)my_i * sdo.t + 8 * half;
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      qf[s] = ld8<E>(qp + 16 * s);
      gf[s] = ld8<E>(gp + 16 * s);
    }
    lrow = Lg[b * sl.b + h * sl.h + (int64_t)my_i * sl.t] * kLog2e;
    // delta: the lane's 16-byte chunks c = 2 s + half, each an fma chain as in
    // fa2_bwd_delta_half_kernel, then that kernel's xor tree over chunks (offsets HS/16 .. 2
    // pair chunks s and s ^ off/2 of this lane; offset 1 pairs the two wave halves).
    const E* op = Og + b * so.b + h * so.h + (int64_t)my_i * so.t + 8 * half;
    float part[QS];
#pragma unroll
    for (int s = 0; s < QS; ++s) {
      const vec8_t<E> o = ld8<E>(op + 16 * s);
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf((float)o[e], (float)gf[s][e], acc);
      part[s] = acc;
    }
#pragma unroll
    for (int off2 = QS / 2; off2 >= 1; off2 >>= 1)
#pragma unroll
      for (int s = 0; s < off2; ++s) part[s] = part[s] + part[s + off2];
    drow = part[0];
  } else {
#pragma unroll
    for (int s = 0; s < QS; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) { qf[s][j] = (E)0.0f; gf[s][j] = (E)0.0f; }
  }
  // The cross-half step of the delta sum; every lane takes part (rows past T sum nothing).
  drow = drow + xor32(drow);
  if (my_i < T && half == 0) delta[(int64_t)bh * T + my_i] = drow;
  // The row loads are complete before the stage loop on every path into it (the compiler
  // would otherwise wait for them inside each stage, draining the next stage's loads too).
  vm_wait_all();

  f32x16 acc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) acc[d] = zero16();

  const int kv_end = CAUSAL ? min(T, (qt + 1) * BM) : T;
  const int n_stages = (kv_end + BN - 1) / BN;

  // K: a task is rows 2 rp and 2 rp + 1 of one 16-byte chunk, stored row-wise and transposed
  // (the two rows' values for one d as one 32-bit word; a wave's 64 tasks are 32 row pairs x 2
  // chunks, so each transposed store hits 64 distinct banks).  hs = 32 has 128 tasks: waves 0
  // and 1 take them (wave-uniform).  V: task c = tid + 256 u is row c / CH, chunk c % CH.
  // Rows of a stage are read through buffer resources over its valid rows; keys past T read
  // as zero and are masked to P = 0.
  u32x4 kst[2 * KL], vst[VLOADS];
  auto pair_of = [&](int u2, int& rp, int& ch) {
    rp = lane & 31;
    ch = 2 * (wave + 4 * u2) + (lane >> 5);
    return KPAIRS % 256 == 0 || ch < CH;
  };
  auto gload = [&](int stage) {
    const int j0 = stage * BN;
    const int rows = min(BN, T - j0);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc16(Kb + (int64_t)j0 * sk.t, rows, sk.t, HS);
    const __amdgpu_buffer_rsrc_t rv = rows_rsrc16(Vb + (int64_t)j0 * sv.t, rows, sv.t, HS);
#pragma unroll
    for (int u2 = 0; u2 < KL; ++u2) {
      int rp, ch;
      if (!pair_of(u2, rp, ch)) continue;
#pragma unroll
      for (int e = 0; e < 2; ++e)
        kst[2 * u2 + e] = ld16_buffer(rk, ((2 * rp + e) * (int)sk.t + 8 * ch) * 2);
    }
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      const int c = tid + 256 * u;
      vst[u] = ld16_buffer(rv, ((c / CH) * (int)sv.t + 8 * (c % CH)) * 2);
    }
  };
  auto lstore = [&](int buf) {
    E* kr = smem + buf * STAGE;
    E* vr = kr + RTILE;
    E* kt = vr + RTILE;
#pragma unroll
    for (int u2 = 0; u2 < KL; ++u2) {
      int rp, ch;
      if (!pair_of(u2, rp, ch)) continue;
      const u32x4 e0 = kst[2 * u2], e1 = kst[2 * u2 + 1];
      *reinterpret_cast<u32x4*>(kr + (2 * rp) * RP + 8 * ch) = e0;
      *reinterpret_cast<u32x4*>(kr + (2 * rp + 1) * RP + 8 * ch) = e1;
      uint32_t* col2 = reinterpret_cast<uint32_t*>(kt + kt_pos(2 * rp));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        col2[(8 * ch + 2 * t) * (TP / 2)] = pack_lo16(e0[t], e1[t]);
        col2[(8 * ch + 2 * t + 1) * (TP / 2)] = pack_hi16(e0[t], e1[t]);
      }
    }
#pragma unroll
    for (int u = 0; u < VLOADS; ++u) {
      const int c = tid + 256 * u;
      *reinterpret_cast<u32x4*>(vr + (c / CH) * RP + 8 * (c % CH)) = vst[u];
    }
  };

  const bool down = CAUSAL && qt < n_qtiles - 1 - qt;  // the short tile of a pair
  auto stage_at = [&](int i) { return down ? n_stages - 1 - i : i; };
  gload(stage_at(0));
  lstore(0);
  __syncthreads();

  for (int i = 0; i < n_stages; ++i) {
    const int s_idx = stage_at(i);
    const int buf = i & 1;
    if (i + 1 < n_stages) gload(stage_at(i + 1));
    const E* kr = smem + buf * STAGE;
    const E* vr = kr + RTILE;
    const E* kt = vr + RTILE;
    if constexpr (CAUSAL && HS == 64) {
      // Both tiles' S and dP chains first (four independent MFMA chains), then their softmax
      // and dQ products.  A/B in one process, same bits: backward +3% causal at hs 64; -2%
      // non-causal and -5% at hs 32, which keep one tile at a time.
      f32x16 sacc2[NSUB], pacc2[NSUB];
      bool live2[NSUB];
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const int jj0 = s_idx * BN + sub * 32;
        live2[sub] = jj0 < T && !(CAUSAL && jj0 > i0 + 31);
        sacc2[sub] = zero16();
#pragma unroll
        for (int r = 0; r < 16; ++r) pacc2[sub][r] = -drow;
        if (!live2[sub]) continue;
        const E* krow = kr + (sub * 32 + col) * RP + 8 * half;
        const E* vrow = vr + (sub * 32 + col) * RP + 8 * half;
#pragma unroll
        for (int s = 0; s < QS; ++s)
          sacc2[sub] = Half16<E>::mfma(ld8<E>(krow + 16 * s), qf[s], sacc2[sub]);
#pragma unroll
        for (int s = 0; s < QS; ++s)
          pacc2[sub] = Half16<E>::mfma(ld8<E>(vrow + 16 * s), gf[s], pacc2[sub]);
      }
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        if (!live2[sub]) continue;
        const int jj0 = s_idx * BN + sub * 32;
        f32x16& sacc = sacc2[sub];
        const f32x16& pacc = pacc2[sub];
        auto exp_scores = [&]<bool MASKED>() {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float x = fmaf(sacc[r], scale_log2, -lrow);
            if (MASKED) {
              const int j = jj0 + mfma_row(r, half);
              if ((CAUSAL && j > my_i) || j >= T) x = -INFINITY;
            }
            sacc[r] = fast_exp2(x);
          }
        };
        if ((CAUSAL && jj0 + 31 > i0) || (jj0 + 32 > T))
          exp_scores.template operator()<true>();
        else
          exp_scores.template operator()<false>();
        vec8_t<E> db[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) db[r >> 3][r & 7] = (E)(sacc[r] * pacc[r]);
#pragma unroll
        for (int d = 0; d < HS / 32; ++d) {
          const E* ktrow = kt + (d * 32 + col) * TP + sub * 32 + 8 * half;
#pragma unroll
          for (int s = 0; s < 2; ++s) acc[d] = Half16<E>::mfma(ld8<E>(ktrow + 16 * s), db[s], acc[d]);
        }
      }
    } else {
#pragma unroll
      for (int sub = 0; sub < NSUB; ++sub) {
        const int jj0 = s_idx * BN + sub * 32;
        if (jj0 >= T) continue;                 // ragged tail
        if (CAUSAL && jj0 > i0 + 31) continue;  // tile entirely above this wave's diagonal

        // S^T and dP^T - delta: lane holds query my_i, keys jj0 + R(r, half).
        f32x16 sacc = zero16(), pacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) pacc[r] = -drow;
        const E* krow = kr + (sub * 32 + col) * RP + 8 * half;
        const E* vrow = vr + (sub * 32 + col) * RP + 8 * half;
#pragma unroll
        for (int s = 0; s < QS; ++s) sacc = Half16<E>::mfma(ld8<E>(krow + 16 * s), qf[s], sacc);
#pragma unroll
        for (int s = 0; s < QS; ++s) pacc = Half16<E>::mfma(ld8<E>(vrow + 16 * s), gf[s], pacc);

        // P = e^{S - L}; masked keys (causal, past T) exactly 0.  Two explicit paths: left to
        // the compiler, the masked form is if-converted into selects on every tile.
        auto exp_scores = [&]<bool MASKED>() {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float x = fmaf(sacc[r], scale_log2, -lrow);
            if (MASKED) {
              const int j = jj0 + mfma_row(r, half);
              if ((CAUSAL && j > my_i) || j >= T) x = -INFINITY;  // 2^x = 0
            }
            sacc[r] = fast_exp2(x);
          }
        };
        if ((CAUSAL && jj0 + 31 > i0) || (jj0 + 32 > T))
          exp_scores.template operator()<true>();
        else
          exp_scores.template operator()<false>();

        // dS = P (dP - delta), rounded to 16 bits as the B operand of dQ^T += K^T dS^T.
        vec8_t<E> db[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) db[r >> 3][r & 7] = (E)(sacc[r] * pacc[r]);
#pragma unroll
        for (int d = 0; d < HS / 32; ++d) {
          const E* ktrow = kt + (d * 32 + col) * TP + sub * 32 + 8 * half;
#pragma unroll
          for (int s = 0; s < 2; ++s) acc[d] = Half16<E>::mfma(ld8<E>(ktrow + 16 * s), db[s], acc[d]);
        }
      }
    }

    if (i + 1 < n_stages) lstore(buf ^ 1);
    __syncthreads();
  }

  if (my_i < T) {
    E* op = dQ + ((int64_t)bh * T + my_i) * HS;
#pragma unroll
    for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        E q4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) q4[e] = (E)(acc[d][4 * g + e] * scale);
        *reinterpret_cast<uint2*>(op + d * 32 + 8 * g + 4 * half) =
            *reinterpret_cast<const uint2*>(q4);
      }
    }
  }
  }  // pass: the stage loop ended on a barrier, so the next pass may refill LDS
}

RowStridesH rsh(const int64_t* s) { return RowStridesH{s[0], s[1], s[2]}; }

bool layout_half_ok(const void* p, const int64_t* s) {
  return p != nullptr && s != nullptr && aligned16(p) && s[3] == 1 && s[0] % 8 == 0 &&
         s[1] % 8 == 0 && s[2] % 8 == 0 && s[2] >= 0 && s[2] < (int64_t(1) << 24);
}

template <typename F>
void dispatch_half(int64_t hs, int causal, F&& f) {
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

int64_t bwd_half_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs, int causal) {
  if (B <= 0 || nh <= 0 || T <= 0 || (hs != 32 && hs != 64 && hs != 128)) return 0;
  return B * nh * ds_tiles_per_head(T, causal != 0) * kDsTileHalf * 2;
}

// The entry points' shared body; `what` names the element type in error messages.
template <class E>
int bwd_half(const uint16_t* q, const int64_t* q_strides, const uint16_t* k,
             const int64_t* k_strides, const uint16_t* v, const int64_t* v_strides,
             const uint16_t* o, const int64_t* o_strides, const uint16_t* d_o,
             const int64_t* do_strides, const float* l, const int64_t* l_strides, int64_t B,
             int64_t nh, int64_t T, int64_t hs, int causal, uint16_t* dq, uint16_t* dk,
             uint16_t* dv, float* delta, void* workspace, int64_t workspace_bytes, void* stream,
             const char* what) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (!layout_half_ok(q, q_strides) || !layout_half_ok(k, k_strides) ||
      !layout_half_ok(v, v_strides) || !layout_half_ok(o, o_strides) ||
      !layout_half_ok(d_o, do_strides))
    return fail(CTA_ERR_LAYOUT, std::string("flash_attention_bwd (") + what +
                                    ") needs unit d-stride, strides divisible by 8, time "
                                    "strides below 2^24 and 16-byte aligned Q/K/V/O/dO");
  if (!l || !l_strides || !delta) return fail(CTA_ERR_INVALID_ARGUMENT, "null L or delta pointer");
  if (!dq || !dk || !dv || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) ||
      !aligned16(workspace))
    return fail(CTA_ERR_LAYOUT, "dQ/dK/dV and the workspace must be 16-byte aligned pointers");
  // Without a workspace that holds one head's dS tiles, the dQ stage recomputes S and dP (the
  // reference's schedule): no O(T^2) memory at any T.
  const int64_t head_bytes = bwd_half_workspace(1, 1, T, hs, causal);
  const bool stored = workspace != nullptr && workspace_bytes >= head_bytes;
  const auto* qb = reinterpret_cast<const E*>(q);
  const auto* kb = reinterpret_cast<const E*>(k);
  const auto* vb = reinterpret_cast<const E*>(v);
  const auto* ob = reinterpret_cast<const E*>(o);
  const auto* gb = reinterpret_cast<const E*>(d_o);
  auto* dqb = reinterpret_cast<E*>(dq);
  auto* dkb = reinterpret_cast<E*>(dk);
  auto* dvb = reinterpret_cast<E*>(dv);
  auto* wsb = reinterpret_cast<E*>(workspace);
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const RowStridesH sl{l_strides[0], l_strides[1], l_strides[2]};
  const int BH = (int)(B * nh);
  hipStream_t st = as_stream(stream);

  const int n_tiles = (int)((T + 127) / 128);
  if (!stored) {
    // Recompute: dQ first (it forms delta and writes it), then dK/dV, which reads it.
    dispatch_half(hs, causal, [&]<int HS, bool C>() {
      const int64_t items = (int64_t)(C ? (n_tiles + 1) / 2 : n_tiles) * BH;
      // waves per SIMD the registers allow (150 / 228 / 356 VGPRs at hs 32 / 64 / 128)
      const int lq = C ? lpt_heads(BH, n_tiles, 4, HS == 32 ? 3 : HS == 64 ? 2 : 1) : 0;
      hipLaunchKernelGGL((fa2_bwd_dq_half_kernel<E, HS, C>),
                         dim3(lq > 0 ? (unsigned)(BH * n_tiles) : xcd_grid(items)), dim3(256), 0,
                         st, qb, kb, vb, gb, ob, l, delta, dqb, (int)nh, (int)T, BH, n_tiles,
                         rsh(q_strides), rsh(k_strides), rsh(v_strides), rsh(do_strides),
                         rsh(o_strides), sl, scale, scale * kLog2e, lq);
      using Cfg = DkdvHalfCfg<HS, C>;
      const int n_ktiles = (int)((T + 32 * Cfg::WAVES - 1) / (32 * Cfg::WAVES));
      const int64_t kitems = (int64_t)(C ? (n_ktiles + 1) / 2 : n_ktiles) * BH;
      hipLaunchKernelGGL(
          (fa2_bwd_dkdv_half_kernel<E, HS, C, Cfg::WAVES, Cfg::BN, Cfg::MINW, false>),
          dim3(xcd_grid(kitems)), dim3(64 * Cfg::WAVES), 0, st, qb, kb, vb, gb, l, delta, dkb,
          dvb, nullptr, (int)nh, (int)T, 0, BH, n_ktiles, rsh(q_strides), rsh(k_strides),
          rsh(v_strides), rsh(do_strides), sl, scale, scale * kLog2e);
    });
    return check_launch("flash_attention_bwd (16-bit, recompute)");
  }

  const int64_t rows = B * nh * T;
  const unsigned dgrid = (unsigned)((rows * (hs / 8) + 255) / 256);
  if (hs == 32)
    hipLaunchKernelGGL((fa2_bwd_delta_half_kernel<E, 32>), dim3(dgrid), dim3(256), 0, st, ob, gb,
                       delta, (int)nh, (int)T, rows, rsh(o_strides), rsh(do_strides));
  else if (hs == 64)
    hipLaunchKernelGGL((fa2_bwd_delta_half_kernel<E, 64>), dim3(dgrid), dim3(256), 0, st, ob, gb,
                       delta, (int)nh, (int)T, rows, rsh(o_strides), rsh(do_strides));
  else
    hipLaunchKernelGGL((fa2_bwd_delta_half_kernel<E, 128>), dim3(dgrid), dim3(256), 0, st, ob, gb,
                       delta, (int)nh, (int)T, rows, rsh(o_strides), rsh(do_strides));
  if (int rc = check_launch("flash_attention_bwd (16-bit) delta")) return rc;

  // Chunks of equal head counts that fit the workspace.
  const int64_t fit = std::min<int64_t>(BH, workspace_bytes / head_bytes);
  const int64_t n_chunks = (BH + fit - 1) / fit;
  const int chunk = (int)((BH + n_chunks - 1) / n_chunks);
  for (int h0 = 0; h0 < BH; h0 += chunk) {
    const int n = std::min(chunk, BH - h0);
    dispatch_half(hs, causal, [&]<int HS, bool C>() {
      using Cfg = DkdvHalfCfg<HS, C>;
      const int n_ktiles = (int)((T + 32 * Cfg::WAVES - 1) / (32 * Cfg::WAVES));
      const int64_t kitems = (int64_t)(C ? (n_ktiles + 1) / 2 : n_ktiles) * n;
      hipLaunchKernelGGL((fa2_bwd_dkdv_half_kernel<E, HS, C, Cfg::WAVES, Cfg::BN, Cfg::MINW, true>),
                         dim3(xcd_grid(kitems)), dim3(64 * Cfg::WAVES), 0, st, qb, kb, vb, gb, l,
                         delta, dkb, dvb, wsb, (int)nh, (int)T, h0, n, n_ktiles,
                         rsh(q_strides), rsh(k_strides), rsh(v_strides), rsh(do_strides), sl,
                         scale, scale * kLog2e);
      const int64_t items = (int64_t)(C ? (n_tiles + 1) / 2 : n_tiles) * n;
      // waves per SIMD (76 / 100 / 180 VGPRs at hs 32 / 64 / 128; LDS allows four)
      const int lq = C ? lpt_heads(n, n_tiles, 4, HS == 128 ? 2 : 4) : 0;
      hipLaunchKernelGGL((fa2_bwd_dq_ds_half_kernel<E, HS, C>),
                         dim3(lq > 0 ? (unsigned)(n * n_tiles) : xcd_grid(items)), dim3(256), 0,
                         st, kb, wsb, dqb, (int)nh, (int)T, h0, n, n_tiles, rsh(k_strides), scale,
                         lq);
    });
    if (int rc = check_launch("flash_attention_bwd (16-bit)")) return rc;
  }
  return CTA_OK;
}

}  // namespace
}  // namespace cta

using namespace cta;

extern "C" int64_t cta_flash_attention_bwd_bf16_workspace(int64_t B, int64_t nh, int64_t T,
                                                          int64_t hs, int causal) {
  return bwd_half_workspace(B, nh, T, hs, causal);
}

extern "C" int cta_flash_attention_bwd_bf16(
    const uint16_t* q, const int64_t* q_strides, const uint16_t* k, const int64_t* k_strides,
    const uint16_t* v, const int64_t* v_strides, const uint16_t* o, const int64_t* o_strides,
    const uint16_t* d_o, const int64_t* do_strides, const float* l, const int64_t* l_strides,
    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal, uint16_t* dq, uint16_t* dk,
    uint16_t* dv, float* delta, void* workspace, int64_t workspace_bytes, void* stream) {
  return bwd_half<__bf16>(q, q_strides, k, k_strides, v, v_strides, o, o_strides, d_o,
                          do_strides, l, l_strides, B, nh, T, hs, causal, dq, dk, dv, delta,
                          workspace, workspace_bytes, stream, "bfloat16");
}

extern "C" int64_t cta_flash_attention_bwd_f16_workspace(int64_t B, int64_t nh, int64_t T,
                                                         int64_t hs, int causal) {
  return bwd_half_workspace(B, nh, T, hs, causal);
}

extern "C" int cta_flash_attention_bwd_f16(
    const uint16_t* q, const int64_t* q_strides, const uint16_t* k, const int64_t* k_strides,
    const uint16_t* v, const int64_t* v_strides, const uint16_t* o, const int64_t* o_strides,
    const uint16_t* d_o, const int64_t* do_strides, const float* l, const int64_t* l_strides,
    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal, uint16_t* dq, uint16_t* dk,
    uint16_t* dv, float* delta, void* workspace, int64_t workspace_bytes, void* stream) {
  return bwd_half<_Float16>(q, q_strides, k, k_strides, v, v_strides, o, o_strides, d_o,
                            do_strides, l, l_strides, B, nh, T, hs, causal, dq, dk, dv, delta,
                            workspace, workspace_bytes, stream, "float16");
}
