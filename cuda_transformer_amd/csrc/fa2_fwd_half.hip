// FlashAttention-2 forward with 16-bit (BF16 or FP16) Q, K, V and FP32 accumulation, CDNA4
// MFMA (v_mfma_f32_32x32x16_bf16 / _f16).  Written for BF16; the FP16 instance differs only in
// the element type and the MFMA (Half16<E>).
//
// The reduced-precision variant the reference lists on its roadmap (README.md:277); the
// semantics are those of the FP32 forward (Transformer_kernels/flash_attention.cuh:27-170):
// O = softmax(s Q K^T) V with s = 1/sqrt(hs), the causal mask j > i, and L = m + ln l in FP32.
// O is written in the input type, L in FP32.  Scores, the online-softmax statistics and the O
// accumulator are FP32; the probabilities are rounded to the input type as the P V operand, as
// in every 16-bit FlashAttention.
//
// gfx950 design (the FP32 kernel's layout trick carried to the 16-deep 16-bit MFMA):
//  * Workgroup = 128 query rows (4 waves x 32), K/V stages of 64 keys (two 32-key tiles),
//    global -> registers -> LDS, double buffered, one barrier per stage.  Causal workgroups
//    take query-tile pairs (n-1-p, p), head-major and XCD-contiguous, and the second pass walks
//    its stages downward, exactly as the FP32 forward.
//  * S^T = K Q^T: lane l supplies K[key l%32][8 (l/32) + 16 s + 0..7] (one 16-byte LDS read of
//    a [key][d] image) and its own query row's q values from registers.  The 32x32 output puts
//    one query per lane: lane l holds the scores of query l%32 for keys R(r, l/32),
//    R(r, h) = 8 (r/4) + 4 h + r%4.
//  * O^T += V^T P^T: for MFMA step s the B operand is the lane's registers r = 8s .. 8s+7,
//    rounded to 16 bits, i.e. keys 16 s + 8 (j/4) + 4 h + j%4 for element j.  V is stored in LDS
//    transposed, [d][key], with bits 2 and 3 of the key index swapped (kt_pos), so those eight
//    keys are adjacent and the A operand is one 16-byte read.
//  * Online softmax, lazy rescaling and the two-half max / sum exchange are the FP32 kernel's.
#include "cta_common.hpp"

namespace cta {
namespace {

struct RowStridesB {
  int64_t b, h, t;  // element strides of the batch, head and time axes (d-stride is 1)
};

template <class E, int HS, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void fa2_fwd_half_kernel(
    const E* __restrict__ Q, const E* __restrict__ K, const E* __restrict__ V,
    E* __restrict__ O, float* __restrict__ L, int nh, int T, int BH, int n_qtiles,
    RowStridesB sq, RowStridesB sk, RowStridesB sv, float scale_log2, int heads_per_xcd = 0) {
  constexpr float kRescaleGap = 8.0f;  // log2 units: probabilities stay below 2^8
  constexpr int BN = 64;             // keys per stage
  constexpr int NSUB = BN / 32;      // 32-key score tiles per stage
  constexpr int BM = 128;
  constexpr int KP = HS + 8;         // bf16 pitch of a K row: conflict-free 16-byte row reads
  constexpr int VP = BN + 8;         // bf16 pitch of a V^T row (one d, every key of the stage)
  constexpr int KTILE = BN * KP;
  constexpr int VTILE = HS * VP;
  constexpr int CH = HS / 8;         // 16-byte chunks per K / V row
  constexpr int LOADS = BN * CH / 256;
  constexpr int QS = HS / 16;        // MFMA steps of S over d
  static_assert(BN * CH % 256 == 0, "stage must split evenly over 256 threads");
  __shared__ __attribute__((aligned(16))) E smem[2 * (KTILE + VTILE)];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
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

  const E* Qb = Q + b * sq.b + h * sq.h;
  const E* Kb = K + b * sk.b + h * sk.h;
  const E* Vb = V + b * sv.b + h * sv.h;

  const int n_pass = qb >= 0 ? 2 : 1;
  for (int pass = 0; pass < n_pass; ++pass) {
  const int qt = pass == 0 ? qa : qb;
  const int i0 = qt * BM + wave * 32;
  const int my_i = i0 + col;

  // This lane's query row, d = 16 s + 8 half + 0..7 for step s.
  vec8_t<E> qf[QS];
  if (my_i < T) {
    const E* qp = Qb + (int64_t)my_i * sq.t + 8 * half;
#pragma unroll
    for (int s = 0; s < QS; ++s) qf[s] = *reinterpret_cast<const vec8_t<E>*>(qp + 16 * s);
  } else {
#pragma unroll
    for (int s = 0; s < QS; ++s)
#pragma unroll
      for (int j = 0; j < 8; ++j) qf[s][j] = (E)0.0f;
  }

  f32x16 oacc[HS / 32];
#pragma unroll
  for (int d = 0; d < HS / 32; ++d) oacc[d] = zero16();
  // Exponent offset of row my_i in log2 units (scores times s log2(e)), lazily updated: it only
  // moves when some row of the wave sees a score more than kRescaleGap above it, so every
  // probability stays below 2^kRescaleGap against the offset in use.
  float mb = -INFINITY;
  float l_run = 0.0f;  // this lane's partial row sum

  const int kv_end = CAUSAL ? min(T, (qt + 1) * BM) : T;
  const int n_stages = (kv_end + BN - 1) / BN;

  // K: thread task c = tid + 256 u is row c / CH, 16-byte chunk c % CH, stored row-wise (eight
  // lanes fill one 128-byte row).  V: a task is rows 2 rp and 2 rp + 1 of one chunk, stored
  // transposed, the two rows' values for one d as one 32-bit word (kt_pos keeps them adjacent).
  // A wave's 64 V tasks are 32 row pairs x 2 chunks, so each transposed store instruction hits
  // 64 distinct banks: the 32 pair positions, and the two chunks' d rows 16 rows (32 banks) apart.
  // hs = 32 has 128 V tasks for 256 threads: waves 0 and 1 take them (ch < CH, wave-uniform).
  static_assert(BN == 64, "32 row pairs per stage");
  constexpr int VPAIRS = 32 * CH;                 // V row-pair tasks per stage
  constexpr int VL = (VPAIRS + 255) / 256;        // ... per thread
  u32x4 kst[LOADS], vst[2 * VL];
  auto vtask = [&](int u2, int& rp, int& ch) {
    rp = lane & 31;
    ch = 2 * (wave + 4 * u2) + (lane >> 5);
    return VPAIRS % 256 == 0 || ch < CH;
  };
  // K/V rows of a stage through buffer resources over its valid rows (scalar base and extent,
  // the same lane offsets every stage).  Rows past T read as zero: those keys are masked to
  // P = 0, so they never reach O.  A stage's 64 rows fit 32-bit offsets (time strides below
  // 2^23, checked on the host).
  auto gload = [&](int stage) {
    const int j0 = stage * BN;
    const int rows = min(BN, T - j0);
    const __amdgpu_buffer_rsrc_t rk = rows_rsrc16(Kb + (int64_t)j0 * sk.t, rows, sk.t, HS);
    const __amdgpu_buffer_rsrc_t rv = rows_rsrc16(Vb + (int64_t)j0 * sv.t, rows, sv.t, HS);
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int c = tid + 256 * u;
      kst[u] = ld16_buffer(rk, ((c / CH) * (int)sk.t + 8 * (c % CH)) * 2);
    }
#pragma unroll
    for (int u2 = 0; u2 < VL; ++u2) {
      int rp, ch;
      if (!vtask(u2, rp, ch)) continue;
#pragma unroll
      for (int e = 0; e < 2; ++e)
        vst[2 * u2 + e] = ld16_buffer(rv, ((2 * rp + e) * (int)sv.t + 8 * ch) * 2);
    }
  };
  auto lstore = [&](int buf) {
    E* ks = smem + buf * (KTILE + VTILE);
    E* vt = ks + KTILE;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int c = tid + 256 * u;
      *reinterpret_cast<u32x4*>(ks + (c / CH) * KP + 8 * (c % CH)) = kst[u];
    }
#pragma unroll
    for (int u2 = 0; u2 < VL; ++u2) {
      int rp, ch;
      if (!vtask(u2, rp, ch)) continue;
      const u32x4 e0 = vst[2 * u2], e1 = vst[2 * u2 + 1];
      uint32_t* col2 = reinterpret_cast<uint32_t*>(vt + kt_pos(2 * rp));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        // d = 8 ch + 2t and 8 ch + 2t + 1: low halves of e0/e1 hold the even d
        col2[(8 * ch + 2 * t) * (VP / 2)] = pack_lo16(e0[t], e1[t]);
        col2[(8 * ch + 2 * t + 1) * (VP / 2)] = pack_hi16(e0[t], e1[t]);
      }
    }
  };

  // One online-softmax step over score tile x0, and x1 too when `two`:
  // replaces the raw scores by their probabilities against the row's offset and adds them to
  // l_run, rescaling l_run and O when the offset moves.  The max is taken over the exponent
  // arguments fma(x, s log2(e), -offset), which the exponentials need anyway; as results of
  // arithmetic they are canonical, so the compiler forms v_max3 trees without canonicalising
  // every MFMA output first.  The first tile of a row (offset -inf) always sets the offset;
  // every processed tile holds at least one unmasked key per row, so it ends finite.
  auto softmax_step = [&]<bool two>(f32x16& x0, f32x16& x1) {
    const float mb0 = mb == -INFINITY ? 0.0f : mb;
    constexpr int NT = two ? 32 : 16;
    float t[NT];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x0[r] = fmaf(x0[r], scale_log2, -mb0);
      t[r] = x0[r];
      if constexpr (two) {
        x1[r] = fmaf(x1[r], scale_log2, -mb0);
        t[16 + r] = x1[r];
      }
    }
    const float my = max_halves(max3_tree(t));
    if (__any(mb == -INFINITY || my > kRescaleGap)) {
      const float mb_new = fmaxf(mb, mb0 + my);
      const float alpha = fast_exp2(mb - mb_new);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < HS / 32; ++d) oacc[d] *= alpha;
      const float shift = mb_new - mb0;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x0[r] -= shift;
        if (two) x1[r] -= shift;
      }
      mb = mb_new;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      x0[r] = fast_exp2(x0[r]);
      if (two) x1[r] = fast_exp2(x1[r]);
      t[r] = two ? x0[r] + x1[r] : x0[r];
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
      for (int r = 0; r < w; ++r) t[r] += t[r + w];
    l_run += t[0];
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
    const E* ks = smem + buf * (KTILE + VTILE);
    const E* vt = ks + KTILE;

    // Causal, hs = 64, and all 64 keys of the stage exist and lie at or below every row of
    // this wave: both 32-key tiles go through one softmax step (one max exchange and one
    // rescale check per 64 keys, two independent MFMA chains in every phase).  It needs ~160
    // VGPRs, which the causal kernel's 3 waves per SIMD allow.  The non-causal kernel fits in
    // 128 VGPRs with one tile at a time, and the fourth wave per SIMD is worth more (measured
    // 869 against 803 TFLOP/s at B4 H32 N4096); so is hs = 128's register budget.
    const bool joint = CAUSAL && HS == 64 && s_idx * BN + BN <= T && s_idx * BN + BN - 1 <= i0;
    if (joint) {
      f32x16 sa = zero16(), sb = zero16();
      const E* krow = ks + col * KP + 8 * half;
#pragma unroll
      for (int s = 0; s < QS; ++s) {
        sa = Half16<E>::mfma(ld8<E>(krow + 16 * s), qf[s], sa);
        sb = Half16<E>::mfma(ld8<E>(krow + 32 * KP + 16 * s), qf[s], sb);
      }
      softmax_step.template operator()<true>(sa, sb);
      vec8_t<E> pa[2], pb[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        pa[r >> 3][r & 7] = (E)sa[r];
        pb[r >> 3][r & 7] = (E)sb[r];
      }
#pragma unroll
      for (int d = 0; d < HS / 32; ++d) {
        const E* vrow = vt + (d * 32 + col) * VP + 8 * half;
#pragma unroll
        for (int s = 0; s < 2; ++s) oacc[d] = Half16<E>::mfma(ld8<E>(vrow + 16 * s), pa[s], oacc[d]);
#pragma unroll
        for (int s = 0; s < 2; ++s)
          oacc[d] = Half16<E>::mfma(ld8<E>(vrow + 32 + 16 * s), pb[s], oacc[d]);
      }
    } else {
#pragma unroll
    for (int sub = 0; sub < NSUB; ++sub) {
      const int jj0 = s_idx * BN + sub * 32;
      if (jj0 >= T) continue;                 // ragged tail
      if (CAUSAL && jj0 > i0 + 31) continue;  // tile entirely above this wave's diagonal

      // S^T tile: sacc[r] = q_{my_i} . k_{jj0 + R(r, half)}
      f32x16 sacc = zero16();
      const E* krow = ks + (sub * 32 + col) * KP + 8 * half;
#pragma unroll
      for (int s = 0; s < QS; ++s)
        sacc = Half16<E>::mfma(*reinterpret_cast<const vec8_t<E>*>(krow + 16 * s), qf[s], sacc);

      const bool need_mask = (CAUSAL && jj0 + 31 > i0) || (jj0 + 32 > T);
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = jj0 + mfma_row(r, half);
          if ((CAUSAL && j > my_i) || j >= T) sacc[r] = -INFINITY;
        }
      }

      softmax_step.template operator()<false>(sacc, sacc);
      vec8_t<E> pf[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) pf[r >> 3][r & 7] = (E)sacc[r];

      // O^T += V^T P^T over the tile's 32 keys, two 16-key MFMA steps per d block.
#pragma unroll
      for (int d = 0; d < HS / 32; ++d) {
        const E* vrow = vt + (d * 32 + col) * VP + sub * 32 + 8 * half;
#pragma unroll
        for (int s = 0; s < 2; ++s)
          oacc[d] = Half16<E>::mfma(*reinterpret_cast<const vec8_t<E>*>(vrow + 16 * s), pf[s], oacc[d]);
      }
    }
    }

    if (i + 1 < n_stages) lstore(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = sum_halves(l_run);
  if (my_i < T) {
    E* op = O + ((int64_t)bh * T + my_i) * HS;
    const float inv = 1.0f / l_tot;
#pragma unroll
    for (int d = 0; d < HS / 32; ++d) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        E o4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o4[e] = (E)(oacc[d][4 * g + e] * inv);
        *reinterpret_cast<uint2*>(op + d * 32 + 8 * g + 4 * half) =
            *reinterpret_cast<const uint2*>(o4);
      }
    }
    if (half == 0) L[(int64_t)bh * T + my_i] = mb * kLn2 + logf(l_tot);
  }
  }  // pass: the K/V loop ended on a barrier, so the next pass may refill LDS
}

template <class E, int HS, bool CAUSAL>
void launch_fwd_half(const E* q, const E* k, const E* v, E* o, float* l, int nh, int T, int BH,
                     RowStridesB sq, RowStridesB sk, RowStridesB sv, float scale,
                     hipStream_t stream) {
  const int n_qtiles = (T + 127) / 128;
  // longest-first tiles on small grids (lpt_heads); waves per SIMD the registers allow (109 /
  // 161 / 218 VGPRs at hs 32 / 64 / 128)
  const int lpt = CAUSAL ? lpt_heads(BH, n_qtiles, 4, HS == 32 ? 4 : HS == 64 ? 3 : 2) : 0;
  const unsigned grid = lpt > 0 ? (unsigned)(BH * n_qtiles)
                                : xcd_grid((int64_t)(CAUSAL ? (n_qtiles + 1) / 2 : n_qtiles) * BH);
  hipLaunchKernelGGL((fa2_fwd_half_kernel<E, HS, CAUSAL>), dim3(grid), dim3(256), 0, stream, q,
                     k, v, o, l, nh, T, BH, n_qtiles, sq, sk, sv, scale * kLog2e, lpt);
}

// 16-bit operands: unit d-stride, (b, h, t) strides divisible by 8 elements, 16-byte aligned,
// time stride in [0, 2^24) (a stage's 64 rows fit 32-bit byte offsets).
bool attn_layout_half_ok(const void* p, const int64_t* s) {
  return p != nullptr && s != nullptr && aligned16(p) && s[3] == 1 && s[0] % 8 == 0 &&
         s[1] % 8 == 0 && s[2] % 8 == 0 && s[2] >= 0 && s[2] < (int64_t(1) << 24);
}

// The entry points' shared body; `what` names the element type in error messages.
template <class E>
int fwd_half(const uint16_t* q, const int64_t* q_strides, const uint16_t* k,
             const int64_t* k_strides, const uint16_t* v, const int64_t* v_strides, int64_t B,
             int64_t nh, int64_t T, int64_t hs, int causal, uint16_t* o, float* l, void* stream,
             const char* what) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (!o || !l) return fail(CTA_ERR_INVALID_ARGUMENT, "null output pointer");
  if (!attn_layout_half_ok(q, q_strides) || !attn_layout_half_ok(k, k_strides) ||
      !attn_layout_half_ok(v, v_strides) || !aligned16(o))
    return fail(CTA_ERR_LAYOUT, std::string("flash_attention_fwd (") + what +
                                    ") needs unit d-stride, strides divisible by 8, time "
                                    "strides below 2^24 and 16-byte aligned Q/K/V/O");
  const RowStridesB sq{q_strides[0], q_strides[1], q_strides[2]};
  const RowStridesB sk{k_strides[0], k_strides[1], k_strides[2]};
  const RowStridesB sv{v_strides[0], v_strides[1], v_strides[2]};
  const float scale = 1.0f / std::sqrt(static_cast<float>(hs));
  const int BH = (int)(B * nh);
  hipStream_t st = as_stream(stream);
  const auto* qb = reinterpret_cast<const E*>(q);
  const auto* kb = reinterpret_cast<const E*>(k);
  const auto* vb = reinterpret_cast<const E*>(v);
  auto* ob = reinterpret_cast<E*>(o);
#define CTA_FWD_HALF(HS_)                                                                     \
  if (causal) launch_fwd_half<E, HS_, true>(qb, kb, vb, ob, l, (int)nh, (int)T, BH, sq, sk,   \
                                            sv, scale, st);                                   \
  else launch_fwd_half<E, HS_, false>(qb, kb, vb, ob, l, (int)nh, (int)T, BH, sq, sk, sv,     \
                                      scale, st);
  if (hs == 32) { CTA_FWD_HALF(32) }
  else if (hs == 64) { CTA_FWD_HALF(64) }
  else { CTA_FWD_HALF(128) }
#undef CTA_FWD_HALF
  return check_launch("flash_attention_fwd (16-bit)");
}

}  // namespace
}  // namespace cta

using namespace cta;

extern "C" int cta_flash_attention_fwd_bf16(const uint16_t* q, const int64_t* q_strides,
                                            const uint16_t* k, const int64_t* k_strides,
                                            const uint16_t* v, const int64_t* v_strides,
                                            int64_t B, int64_t nh, int64_t T, int64_t hs,
                                            int causal, uint16_t* o, float* l, void* stream) {
  return fwd_half<__bf16>(q, q_strides, k, k_strides, v, v_strides, B, nh, T, hs, causal, o, l,
                          stream, "bfloat16");
}

extern "C" int cta_flash_attention_fwd_f16(const uint16_t* q, const int64_t* q_strides,
                                           const uint16_t* k, const int64_t* k_strides,
                                           const uint16_t* v, const int64_t* v_strides,
                                           int64_t B, int64_t nh, int64_t T, int64_t hs,
                                           int causal, uint16_t* o, float* l, void* stream) {
  return fwd_half<_Float16>(q, q_strides, k, k_strides, v, v_strides, B, nh, T, hs, causal, o,
                            l, stream, "float16");
}
