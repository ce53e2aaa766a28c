// Strided, batched FP32 GEMM on CDNA4 MFMA, and the linear layer's C entry points.
//
//   out[z][m][n] = alpha * sum_k A[z][m][k] * B[z][k][n]  (+ bias[n])  (causal: -inf for n > m)
//
// optionally followed by a GELU stage (erf or tanh form) in the epilogue (the GPT MLP's
// fc1 -> GELU forward and fc2 -> GELU backward products, each one pass over the output instead
// of two).
//
// This one kernel backs the reference's fused_multiply_add (Transformer_kernels/
// fused_multiply_add.cuh:10-92, launched from Transformer_launchers/linear_layer.cu:28-70),
// its strided batched cuda_bmm (batched_matrix_multiply.cuh:9-75) and the two GEMM stages of
// the naive attention (causal_self_attention_fwd.cuh:9-127).  Every operand is addressed
// through strides, so transposed views (W^T, x^T in the linear backward) need no copies.
// The batch index z is split as (z / zin, z % zin) with a stride per level, which lets
// the naive attention address heads inside a packed (B, T, 3C) tensor directly.
//
// gfx950 design: workgroup tile 128x128 of four 64x64 waves, or 64x128 of four 32x64 waves for
// narrow outputs, each wave owning a block of v_mfma_f32_32x32x2_f32 tiles.  A and B tiles are
// staged through LDS as [m][k] and [n][k] (k contiguous, pitch BK+4), so each MFMA operand
// fragment is a pair of 16-byte LDS reads whatever the operand's memory order.  Operand loads
// are dwordx4 buffer loads along whichever dimension is contiguous in memory (template mode),
// with scalar loads for irregular strides; the epilogue stores through buffer stores.  Both
// address a tile from scalar bases with fixed per-lane offsets and let the buffer's range check
// zero (loads) or drop (stores) what lies outside the operand, so the K loop and the epilogue
// carry no per-element address arithmetic or bounds tests.  Within a slice the instruction
// order is pinned (sched_group_barrier): operand loads and LDS stores sit between the MFMAs, and
// the next slice's fragments are read while the current slice's last MFMAs run.
//
// This header holds the kernel templates and the per-tile launcher; gemm_tiles_*.hip each
// instantiate a few tile types (gemm_launch_<tile>), so the build compiles them in parallel, and
// gemm.hip picks the tile and holds the C entry points.
#pragma once

#include "cta_common.hpp"
#include "gemm.hpp"

namespace cta {

enum LoadMode { kVecK = 0, kVecMN = 1, kScalar = 2 };

namespace {

// Workgroup tile BM x BN, K-slice BK, WM x WN waves; each wave owns a (BM/WM) x (BN/WN) block of
// 32x32 MFMA tiles.  LDS rows hold one k-slice of one m (or n) index, pitch BK + 4 floats.
template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct GemmTile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int MB = BM / WM / 32;  // MFMA tiles per wave along m
  static constexpr int NB = BN / WN / 32;  // ... along n
  static constexpr int KP = BK + 4;
  static constexpr int LDS_FLOATS = 2 * (BM + BN) * KP;  // double buffered
  static_assert(MB >= 1 && NB >= 1 && BK % 8 == 0, "bad GEMM tile");
};

// Row and k offset of float4 number f of a k-contiguous slice.  Four lanes read one row's 64
// contiguous bytes.  With BK = 16 (LDS pitch 20 floats) a 16-byte LDS write serves 8 lanes =
// 2 rows at once, and rows r and r+4 start 4 bank groups apart: pairing them keeps the 8
// writes on 8 distinct bank groups.
template <int BK>
__device__ __forceinline__ void veck_coords(int f, int& r, int& k4) {
  if (BK == 16) {
    const int g = f >> 3, l = f & 7;
    r = ((g >> 2) << 3) + (g & 3) + ((l >> 2) << 2);
    k4 = (l & 3) * 4;
  } else {
    r = f / (BK / 4);
    k4 = (f % (BK / 4)) * 4;
  }
}

// Loads one ROWS x BK slice of an operand into registers.  `rows` indexes m (A) or n (B); the
// operand is row-major in (row, k) when kVecK, (k, row) when kVecMN.
//
// Vector modes read through buffer loads: each lane's byte offset within a slice is fixed for
// the whole K loop, and each slice only moves the resource's base and extent (scalar work), so
// the loop carries no per-load address arithmetic.  Reads outside the resource return zero,
// which zeroes k past the end of the K range and slices past the last one; rows past R read
// zero (kVecK) or in-bounds values that only feed output rows/columns never stored (kVecMN).
// On a ragged last slice a kVecK lane whose k lies past the end moves its offset out of range.
template <int MODE, int ROWS, int BK, int THREADS>
struct TileLoader {
  static constexpr int LOADS = ROWS * BK / 4 / THREADS;
  static_assert(ROWS * BK % (4 * THREADS) == 0, "tile must split evenly over the workgroup");
  float4 v[LOADS];
};

template <int MODE, int ROWS, int BK, int THREADS>
struct LoadPlan {
  static constexpr int LOADS = TileLoader<MODE, ROWS, BK, THREADS>::LOADS;
  const float* base;  // (row0, k0) of the tile
  int64_t s_row, s_k;
  int rows;           // valid rows from row0: min(ROWS, R - row0) (kVecK) or R - row0 (kVecMN)
  int row0, kb, R, ke;
  int voff[LOADS];    // vector modes: byte offset of the lane's float4 within a slice
  int kq[LOADS];      // kVecK: the float4's k within a slice
  __device__ __forceinline__ void init(const float* b, int64_t sr, int64_t sk, int r0, int k0,
                                       int R_, int K_, int tid) {
    s_row = sr; s_k = sk; row0 = r0; kb = k0; R = R_; ke = K_;
    if (MODE == kVecK) {
      base = b + (int64_t)r0 * sr + k0;
      rows = min(ROWS, R_ - r0);
    } else if (MODE == kVecMN) {
      base = b + (int64_t)k0 * sk + r0;
      rows = R_ - r0;
    } else {
      base = b;
    }
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + THREADS * u;
      if (MODE == kVecMN) {
        const int k = f % BK, r4 = (f / BK) * 4;
        voff[u] = (int)(((int64_t)k * sk + r4) * 4);
        kq[u] = k;
      } else {
        int r, k4;
        veck_coords<BK>(f, r, k4);
        voff[u] = (int)(((int64_t)r * sr + k4) * 4);
        kq[u] = k4;
      }
    }
  }
  // Slice t (k from kb + t BK) into regs.
  __device__ __forceinline__ void load(TileLoader<MODE, ROWS, BK, THREADS>& L, int t,
                                       int tid) const {
    const int k0 = kb + t * BK;
    const int klim = min(BK, ke - k0);  // <= 0 past the end: nothing in range
    if (MODE == kScalar) {
#pragma unroll
      for (int u = 0; u < LOADS; ++u) {
        const int f = tid + THREADS * u;
        int r, k4;
        veck_coords<BK>(f, r, k4);
        const int gr = row0 + r, gk = k0 + k4;
        float t4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          t4[e] = (gr < R && gk + e < ke) ? base[(int64_t)gr * s_row + (int64_t)(gk + e) * s_k] : 0.0f;
        L.v[u] = make_float4(t4[0], t4[1], t4[2], t4[3]);
      }
      return;
    }
    const float* bt;
    int nbytes;
    if (MODE == kVecK) {
      bt = base + (int64_t)t * BK;
      nbytes = klim > 0 ? (int)(((int64_t)(rows - 1) * s_row + klim) * 4) : 0;
    } else {
      bt = base + (int64_t)t * BK * s_k;
      nbytes = klim > 0 ? (int)(((int64_t)(klim - 1) * s_k + rows) * 4) : 0;
    }
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(bt), (short)0, nbytes, 0x00020000);
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int vo = (MODE == kVecMN || kq[u] < klim) ? voff[u] : (int)0x80000000;
      const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, vo, 0, 0);
      L.v[u] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z),
                           __uint_as_float(w.w));
    }
  }
};

// LDS image of a slice in regs: [row][k], pitch BK + 4.
template <int MODE, int ROWS, int BK, int THREADS>
__device__ __forceinline__ void store_slice(const TileLoader<MODE, ROWS, BK, THREADS>& L,
                                            float* lds, int tid) {
  constexpr int KP = BK + 4;
#pragma unroll
  for (int u = 0; u < TileLoader<MODE, ROWS, BK, THREADS>::LOADS; ++u) {
    const int f = tid + THREADS * u;
    const float4 w = L.v[u];
    if (MODE == kVecMN) {
      const int k = f % BK, r4 = (f / BK) * 4;
      lds[(r4 + 0) * KP + k] = w.x;
      lds[(r4 + 1) * KP + k] = w.y;
      lds[(r4 + 2) * KP + k] = w.z;
      lds[(r4 + 3) * KP + k] = w.w;
    } else {
      int r, k4;
      veck_coords<BK>(f, r, k4);
      st4(lds + r * KP + k4, w);
    }
  }
}

// One wave's operand fragments of one K-slice: per MFMA tile row (A) or column (B), KC = BK / 8
// 16-byte chunks, each feeding four MFMAs (lane half h supplies k = 2e + h of chunk element e).
template <class TL>
struct Frags {
  static constexpr int KC = TL::BK / 8;
  float4 a[TL::MB][KC], b[TL::NB][KC];
};

// Reads a slice's fragments from LDS: A rows [BM][KP] then B rows [BN][KP] at `as`.
template <class TL>
__device__ __forceinline__ void read_frags(const float* as, Frags<TL>& f, int wm, int wn,
                                           int half, int col) {
  constexpr int BM = TL::BM, BN = TL::BN, BK = TL::BK, KP = TL::KP, KC = Frags<TL>::KC;
  const float* bs = as + BM * KP;
#pragma unroll
  for (int i = 0; i < TL::MB; ++i) {
    const float* ap = as + (wm * (BM / TL::WM) + i * 32 + col) * KP + half * (BK / 2);
#pragma unroll
    for (int c = 0; c < KC; ++c) f.a[i][c] = ld4(ap + 4 * c);
  }
#pragma unroll
  for (int j = 0; j < TL::NB; ++j) {
    const float* bp = bs + (wn * (BN / TL::WN) + j * 32 + col) * KP + half * (BK / 2);
#pragma unroll
    for (int c = 0; c < KC; ++c) f.b[j][c] = ld4(bp + 4 * c);
  }
}

// The MFMAs of chunks [C0, C1) of a slice, in k order for every accumulator.
template <class TL, int C0, int C1>
__device__ __forceinline__ void mma_chunks(const Frags<TL>& f, f32x16 (&acc)[TL::MB][TL::NB]) {
#pragma unroll
  for (int c = C0; c < C1; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < TL::MB; ++i)
#pragma unroll
        for (int j = 0; j < TL::NB; ++j) {
          const float4 av = f.a[i][c], bv = f.b[j][c];
          const float a = e == 0 ? av.x : e == 1 ? av.y : e == 2 ? av.z : av.w;
          const float b = e == 0 ? bv.x : e == 1 ? bv.y : e == 2 ? bv.z : bv.w;
          acc[i][j] = mfma32(a, b, acc[i][j]);
        }
}

// Instruction order of a slice's first MFMAs (sched_group_barrier masks: 0x008 MFMA,
// 0x020 global load, 0x200 LDS store): one MFMA at a time, the next slice's global loads after
// the first NV of them and its LDS stores, two at a time, after the middle one, so both issue
// while the MFMA pipe is busy instead of between slices.
template <int I, int NM, int NV, int NW>
__device__ __forceinline__ void sched_first_part() {
  if constexpr (I < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (I < NV) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    if constexpr (I >= NM / 2 && (I - NM / 2) * 2 < NW)
      __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
    sched_first_part<I + 1, NM, NV, NW>();
  }
}

// Instruction order of a slice's last MFMAs: all of them in a row, or with CS the column-sum
// adds (NA VALU instructions) one after each of the first MFMAs, where the wave would otherwise
// wait for the matrix pipe.  (The four adds in a row just before the barrier cost the kernel
// 2-4%; one per MFMA here, 0-2%.)
template <int N>
__device__ __forceinline__ void sched_interleave() {
  if constexpr (N > 0) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
    sched_interleave<N - 1>();
  }
}

template <bool CS, int NM, int NA>
__device__ __forceinline__ void sched_second_part() {
  if constexpr (CS) {
    static_assert(NA <= NM, "one add per MFMA");
    sched_interleave<NA>();
    __builtin_amdgcn_sched_group_barrier(0x008, NM - NA, 0);
  } else {
    __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
  }
}

// Stores a wave's block of one output tile.  RAW: the accumulators as they are (split-K
// partials); otherwise alpha, bias, the causal mask (MASK) and the pointwise stage ACT.  `Cz`
// and `Xz` are the batch's output and aux planes, row stride srow.  The block is stored through
// buffer stores from its origin: a lane's column is a fixed per-lane offset (moved out of range
// when the column lies past N), each row's offset is scalar, and rows past M fall outside the
// resource, so the stores need no per-element bounds tests or 64-bit address arithmetic.
// One element of the epilogue: v = alpha * acc + bias, the mask, the gradient stages (xg: the
// aux value), then the value stored to C (cv) and, for the forward GELU stages, to aux (xv).
template <int ACT, bool RAW, bool MASK>
__device__ __forceinline__ void epilogue_value(float a, float bias, float xg,
                                               const GemmEpilogue& ep, bool masked, float& cv,
                                               float& xv) {
  float val = a;
  if (!RAW) {
    val = fmaf(ep.alpha, val, bias);
    if (MASK && masked) val = -INFINITY;
    if constexpr (ACT == kActGeluGrad) val = gelu_grad(xg, val);
    else if constexpr (ACT == kActGeluTanhGrad) val = gelu_tanh_grad(xg, val);
    else if constexpr (ACT == kActMulAux) val = val * xg;
  }
  // The derivative forms store gelu'(v) (its product with g = 1.0 is exact, so a later
  // kActMulAux stage gives gelu_grad(v, g) bit for bit) and gelu(v).
  cv = val;
  if (!RAW && ACT == kActGeluDeriv) cv = gelu_grad(val, 1.0f);
  if (!RAW && ACT == kActGeluTanhDeriv) cv = gelu_tanh_grad(val, 1.0f);
  xv = 0.0f;
  if (!RAW && (ACT == kActGelu || ACT == kActGeluDeriv)) xv = gelu_f(val);
  if (!RAW && (ACT == kActGeluTanh || ACT == kActGeluTanhDeriv)) xv = gelu_tanh_f(val);
}

// The wave's block when it spans 2^31 bytes or more (row strides of 2^22 floats and up), which
// 32-bit buffer offsets cannot address: plain stores through 64-bit addresses with explicit
// row and column bounds, the same values as block_store's.
template <class TL, int ACT, bool RAW, bool MASK>
__device__ __forceinline__ void block_store_wide(const f32x16 (&acc)[TL::MB][TL::NB], float* Cz,
                                              float* Xz, int64_t srow, const GemmEpilogue& ep,
                                              int M, int N, int mw, int nw, int half, int col) {
  constexpr bool kGrad =
      !RAW && (ACT == kActGeluGrad || ACT == kActGeluTanhGrad || ACT == kActMulAux);
  constexpr bool kAux = !RAW && (ACT == kActGelu || ACT == kActGeluDeriv ||
                                 ACT == kActGeluTanh || ACT == kActGeluTanhDeriv);
#pragma unroll
  for (int j = 0; j < TL::NB; ++j) {
    const int n = nw + j * 32 + col;
    if (n >= N) continue;
    const float bias = (!RAW && ep.bias) ? ep.bias[(int64_t)n * ep.bias_stride] : 0.0f;
#pragma unroll
    for (int i = 0; i < TL::MB; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mw + i * 32 + mfma_row(r, half);
        if (m >= M) continue;
        const int64_t at = (int64_t)m * srow + n;
        const float xg = kGrad ? Xz[at] : 0.0f;
        float cv, xv;
        epilogue_value<ACT, RAW, MASK>(acc[i][j][r], bias, xg, ep, n > m, cv, xv);
        Cz[at] = cv;
        if (kAux) Xz[at] = xv;
      }
    }
  }
}

template <class TL, int ACT, bool RAW, bool MASK>
__device__ __forceinline__ void block_store(const f32x16 (&acc)[TL::MB][TL::NB], float* Cz,
                                            float* Xz, int64_t srow, const GemmEpilogue& ep,
                                            int M, int N, int mw, int nw, int half, int col) {
  constexpr int MB = TL::MB, NB = TL::NB;
  constexpr int WROWS = TL::BM / TL::WM, WCOLS = TL::BN / TL::WN;
  constexpr bool kGrad =
      !RAW && (ACT == kActGeluGrad || ACT == kActGeluTanhGrad || ACT == kActMulAux);
  const int64_t span = ((int64_t)(min(WROWS, M - mw) - 1) * srow + min(WCOLS, N - nw)) * 4;
  if (span >= ((int64_t)1 << 31) || (int64_t)WROWS * srow * 4 >= ((int64_t)1 << 31)) {
    block_store_wide<TL, ACT, RAW, MASK>(acc, Cz, Xz, srow, ep, M, N, mw, nw, half, col);
    return;
  }
  float* Cb = Cz + (int64_t)mw * srow + nw;
  float* Xb = Xz ? Xz + (int64_t)mw * srow + nw : Cb;
  const int nbytes = (int)span;
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(Cb, (short)0, nbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(Xb, (short)0, nbytes, 0x00020000);
  const int row_bytes = (int)(srow * 4);
  int vo[NB];
  float bv[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = nw + j * 32 + col;
    bv[j] = (!RAW && ep.bias && n < N) ? ep.bias[(int64_t)n * ep.bias_stride] : 0.0f;
    vo[j] = n < N ? 4 * half * row_bytes + (j * 32 + col) * 4 : (int)0x80000000;
  }
  // The gradient stages read the pre-activations (kActMulAux: the saved derivatives): all of
  // the block's loads are issued before its first store, so their latencies overlap.  Each
  // element's aux value is read before any store, so dx may alias it.
  float xg[kGrad ? MB : 1][kGrad ? NB : 1][16];
  if constexpr (kGrad) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          xg[i][j][r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
              rx, vo[j], (i * 32 + 8 * (r >> 2) + (r & 3)) * row_bytes, 0));
  }
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = nw + j * 32 + col;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int so = (i * 32 + 8 * (r >> 2) + (r & 3)) * row_bytes;
        float cv, xv;
        epilogue_value<ACT, RAW, MASK>(acc[i][j][r], bv[j], kGrad ? xg[i][j][r] : 0.0f, ep,
                                       n > mw + i * 32 + mfma_row(r, half), cv, xv);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(cv), rc, vo[j], so, 0);
        if (!RAW && (ACT == kActGelu || ACT == kActGeluDeriv || ACT == kActGeluTanh ||
                     ACT == kActGeluTanhDeriv))
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(xv), rx, vo[j], so, 0);
      }
    }
  }
}

// split_ws == nullptr: out = alpha * A B (+ bias, mask) written through C.
// split_ws != nullptr: blockIdx.z = s * Z + z covers K range [s*kchunk, (s+1)*kchunk) and the raw
// partial sum goes to split_ws[s][z][m][n] (dense); gemm_splitk_reduce finishes the epilogue.
// CS (Z == 1, B in kVecMN mode): the workgroups of the first row of tiles also sum B's columns
// over their K range, into ep.colsum or, split, into row s of the [S][N] block that follows
// the partial products.
template <class TL, int AMODE, int BMODE, int ACT, bool CS = false>
__global__ __launch_bounds__(TL::THREADS) void gemm_kernel(GemmOperand A, GemmOperand B,
                                                           GemmOut C, GemmEpilogue ep, int M,
                                                           int N, int K, int zin, int Z,
                                                           int kchunk,
                                                           float* __restrict__ split_ws) {
  constexpr int BM = TL::BM, BN = TL::BN, BK = TL::BK, KP = TL::KP;
  constexpr int MB = TL::MB, NB = TL::NB;
  __shared__ __attribute__((aligned(16))) float smem[TL::LDS_FLOATS];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = wave_index();
  const int half = lane >> 5, col = lane & 31;
  const int wm = wave / TL::WN, wn = wave % TL::WN;

  // Without a K split: the output tiles of all batches in one row-major list (batch, m, n; n
  // fastest), each XCD walking a contiguous run of it, so the workgroups that share an A row
  // block run on one XCD and read it into one L2.  Split along K: tile (x, y), z = split * Z +
  // batch.
  int n0, m0, z, split;
  if (split_ws == nullptr) {
    const int ntn = (N + BN - 1) / BN, ntiles = ntn * ((M + BM - 1) / BM);
    const int w = xcd_work_item(blockIdx.x, ntiles * Z);
    if (w >= ntiles * Z) return;
    z = w / ntiles;
    const int t = w - z * ntiles;
    n0 = (t % ntn) * BN;
    m0 = (t / ntn) * BM;
    split = 0;
  } else {
    n0 = blockIdx.x * BN;
    m0 = blockIdx.y * BM;
    z = blockIdx.z % Z;
    split = blockIdx.z / Z;
  }
  const int zo = z / zin, zi = z - zo * zin;
  const float* Ab = A.p + zo * A.s_outer + zi * A.s_inner;
  const float* Bb = B.p + zo * B.s_outer + zi * B.s_inner;
  const int kb = split * kchunk;
  const int ke = min(K, kb + kchunk);

  // A rows are m with (s_row, s_col) = (m, k); B "rows" are n with (n, k) = (s_col, s_row).
  // Global loads run two K-slices ahead of the MFMAs (two register sets, alternating), so a
  // slice's loads have two slices of MFMA work to arrive; LDS is double buffered.  Vector-mode
  // reads past K, or past the last slice, return zero.
  using LA = TileLoader<AMODE, BM, BK, TL::THREADS>;
  using LB = TileLoader<BMODE, BN, BK, TL::THREADS>;
  LoadPlan<AMODE, BM, BK, TL::THREADS> pa;
  LoadPlan<BMODE, BN, BK, TL::THREADS> pb;
  pa.init(Ab, A.s_row, A.s_col, m0, kb, M, ke, tid);
  pb.init(Bb, B.s_col, B.s_row, n0, kb, N, ke, tid);
  LA la0, la1;
  LB lb0, lb1;
  const int nk = (ke - kb + BK - 1) / BK;
  static_assert(!CS || BMODE == kVecMN, "column sums come from n-contiguous B slices");

  // CS: each lane's B float4s hold the same four columns at the same k residue in every slice,
  // so the lane sums them as the slices pass through its registers (slices past the end are
  // zero); the lanes of one column group are combined after the loop.
  float4 cs[CS ? LB::LOADS : 1];
  auto add_cs = [&](const LB& lb) {
    if constexpr (CS) {
#pragma unroll
      for (int u = 0; u < LB::LOADS; ++u) {
        cs[u].x += lb.v[u].x; cs[u].y += lb.v[u].y; cs[u].z += lb.v[u].z; cs[u].w += lb.v[u].w;
      }
    }
  };
#pragma unroll
  for (int u = 0; u < (CS ? LB::LOADS : 1); ++u) cs[u] = zero4();

  f32x16 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = zero16();

  // Slice count rounded up to even: slices past the end read nothing in range, so they are
  // stored as zeros and add nothing.  The loop then has no conditional loads or stores, which
  // keeps the compiler's wait counts exact (a load issued two slices ahead is not waited for
  // until its LDS store).
  const int nk2 = (nk + 1) & ~1;
  pa.load(la0, 0, tid);
  pb.load(lb0, 0, tid);
  pa.load(la1, 1, tid);
  pb.load(lb1, 1, tid);
  store_slice(la0, smem, tid);
  store_slice(lb0, smem + BM * KP, tid);
  add_cs(lb0);
  __syncthreads();

  // Each slice's MFMAs run in two parts around the barrier that publishes the next slice.  The
  // first part carries the next-but-one slice's global loads and the next slice's LDS stores;
  // right after the barrier the wave issues the next slice's fragment reads, which complete
  // under the second part, so no wave waits on LDS latency before its MFMAs.  A buffer is
  // rewritten only after the barrier that follows every wave's reads of it (the barrier waits
  // for outstanding LDS reads).
  constexpr int KC = Frags<TL>::KC;
  static_assert(KC % 2 == 0, "a slice splits into two halves of chunks");
  constexpr int NM1 = MB * NB * 4 * (KC / 2);  // MFMAs per part
  constexpr int NVM = LA::LOADS + LB::LOADS;
  constexpr int NDW = LA::LOADS * (AMODE == kVecMN ? 4 : 1) + LB::LOADS * (BMODE == kVecMN ? 4 : 1);
  constexpr int NDR = (MB + NB) * KC;
  float* const buf0 = smem;
  float* const buf1 = smem + (BM + BN) * KP;
  Frags<TL> f0, f1;
  read_frags<TL>(buf0, f0, wm, wn, half, col);
  for (int t = 0; t < nk2; t += 2) {
    // slice t in f0; slices t+2 (set 0) and t+1 (set 1, stored below) in flight
    pa.load(la0, t + 2, tid);
    pb.load(lb0, t + 2, tid);
    mma_chunks<TL, 0, KC / 2>(f0, acc);
    store_slice(la1, buf1, tid);
    store_slice(lb1, buf1 + BM * KP, tid);
    sched_first_part<0, NM1, NVM, NDW>();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_frags<TL>(buf1, f1, wm, wn, half, col);
    mma_chunks<TL, KC / 2, KC>(f0, acc);
    add_cs(lb1);
    __builtin_amdgcn_sched_group_barrier(0x100, NDR, 0);  // LDS reads first
    sched_second_part<CS, NM1, 4 * LB::LOADS>();
    __builtin_amdgcn_sched_barrier(0);
    // slice t+1 in f1
    pa.load(la1, t + 3, tid);
    pb.load(lb1, t + 3, tid);
    mma_chunks<TL, 0, KC / 2>(f1, acc);
    store_slice(la0, buf0, tid);
    store_slice(lb0, buf0 + BM * KP, tid);
    sched_first_part<0, NM1, NVM, NDW>();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_frags<TL>(buf0, f0, wm, wn, half, col);
    mma_chunks<TL, KC / 2, KC>(f1, acc);
    add_cs(lb0);
    __builtin_amdgcn_sched_group_barrier(0x100, NDR, 0);
    sched_second_part<CS, NM1, 4 * LB::LOADS>();
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (CS) {
    if (m0 == 0) {
      // Lanes f with the same f / BK share a column group (BK consecutive lanes of one wave).
      float* out = split_ws ? split_ws + (int64_t)gridDim.z * M * N + (int64_t)split * N
                            : ep.colsum;
#pragma unroll
      for (int u = 0; u < LB::LOADS; ++u) {
        float4 v = cs[u];
#pragma unroll
        for (int off = 1; off < BK; off <<= 1) {
          v.x += __shfl_xor(v.x, off);
          v.y += __shfl_xor(v.y, off);
          v.z += __shfl_xor(v.z, off);
          v.w += __shfl_xor(v.w, off);
        }
        const int f = tid + TL::THREADS * u;
        const int n = n0 + (f / BK) * 4;
        if (f % BK == 0 && n < N) {  // N % 4 == 0: the whole group is in range
          out[n] = v.x; out[n + 1] = v.y; out[n + 2] = v.z; out[n + 3] = v.w;
        }
      }
    }
  }

  const int mw = m0 + wm * (BM / TL::WM), nw = n0 + wn * (BN / TL::WN);
  if (mw >= M || nw >= N) return;
  // The block's byte extent must fit the 32-bit buffer offsets; the launcher checks it.
  if (split_ws != nullptr) {
    float* Pz = split_ws + ((int64_t)split * Z + z) * M * N;
    block_store<TL, kActNone, true, false>(acc, Pz, nullptr, N, ep, M, N, mw, nw, half, col);
    return;
  }
  float* Cz = C.p + zo * C.s_outer + zi * C.s_inner;
  float* Xz = ep.aux ? ep.aux + zo * C.s_outer + zi * C.s_inner : nullptr;
  if (ep.causal_mask)
    block_store<TL, ACT, false, true>(acc, Cz, Xz, C.s_row, ep, M, N, mw, nw, half, col);
  else
    block_store<TL, ACT, false, false>(acc, Cz, Xz, C.s_row, ep, M, N, mw, nw, half, col);
}

// Fixed-order sum of the split-K partials plus the epilogue of gemm_kernel; with ep.colsum also
// of the per-split column sums stored after them.
__global__ __launch_bounds__(256) void gemm_splitk_reduce(const float* __restrict__ ws, int S,
                                                          int Z, int M, int N, GemmOut C,
                                                          GemmEpilogue ep, int zin) {
  const int64_t total = (int64_t)Z * M * N;
  const int64_t plane = total;
  const int64_t all = total + (ep.colsum ? N : 0);
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < all;
       e += (int64_t)gridDim.x * 256) {
    if (e >= total) {
      const float* p = ws + (int64_t)S * plane + (e - total);
      float t = p[0];
      for (int s = 1; s < S; ++s) t += p[(int64_t)s * N];
      ep.colsum[e - total] = t;
      continue;
    }
    float acc = ws[e];
    for (int s = 1; s < S; ++s) acc += ws[(int64_t)s * plane + e];
    const int64_t z = e / ((int64_t)M * N);
    const int64_t mn = e - z * M * N;
    const int m = (int)(mn / N), n = (int)(mn - (int64_t)m * N);
    const int64_t zo = z / zin, zi = z - zo * zin;
    float val = fmaf(ep.alpha, acc, ep.bias ? ep.bias[(int64_t)n * ep.bias_stride] : 0.0f);
    if (ep.causal_mask && n > m) val = -INFINITY;
    const int64_t off = zo * C.s_outer + zi * C.s_inner + (int64_t)m * C.s_row + n;
    if (ep.act == kActGeluGrad) val = gelu_grad(ep.aux[off], val);
    if (ep.act == kActGeluTanhGrad) val = gelu_tanh_grad(ep.aux[off], val);
    if (ep.act == kActMulAux) val = val * ep.aux[off];
    C.p[off] = ep.act == kActGeluDeriv       ? gelu_grad(val, 1.0f)
               : ep.act == kActGeluTanhDeriv ? gelu_tanh_grad(val, 1.0f)
                                             : val;
    if (ep.act == kActGelu || ep.act == kActGeluDeriv) ep.aux[off] = gelu_f(val);
    if (ep.act == kActGeluTanh || ep.act == kActGeluTanhDeriv) ep.aux[off] = gelu_tanh_f(val);
  }
}

bool vec_ok(const GemmOperand& op, bool contig_is_col) {
  // dwordx4 loads along the contiguous dimension need 16-byte aligned rows.
  const int64_t s_other = contig_is_col ? op.s_row : op.s_col;
  return aligned16(op.p) && s_other % 4 == 0 && op.s_outer % 4 == 0 && op.s_inner % 4 == 0;
}

// Load mode of an operand.  A: (s_row, s_col) = (m, k); B: (k, n).  `rows` is M for A and N for
// B.  The vector modes also need the contiguous extent to be a multiple of 4 (a float4 lies
// wholly inside or outside the operand) and at least 4.
int pick_mode(const GemmOperand& op, bool is_a, int64_t rows, int64_t K) {
  const int64_t s_k = is_a ? op.s_col : op.s_row;
  const int64_t s_mn = is_a ? op.s_row : op.s_col;
  // The buffer loads address a slice with 32-bit byte offsets and rely on rows (kVecK) or
  // k rows (kVecMN) not overlapping, so that reads past the valid range fall outside it.
  constexpr int64_t kMaxBytes = (int64_t)1 << 31;
  if (s_k == 1 && K % 4 == 0 && K >= 4 && vec_ok(op, is_a) && s_mn >= K &&
      (255 * s_mn + 64) * 4 < kMaxBytes)
    return kVecK;
  if (s_mn == 1 && rows % 4 == 0 && rows >= 4 && vec_ok(op, !is_a) && s_k >= rows &&
      (63 * s_k + std::max<int64_t>(rows, 256)) * 4 < kMaxBytes)
    return kVecMN;
  return kScalar;
}

template <class TL, int AM, int ACT, bool CS>
void dispatch_b(int bm, dim3 grid, hipStream_t st, const GemmOperand& A, const GemmOperand& B,
                const GemmOut& C, const GemmEpilogue& ep, int M, int N, int K, int zin, int Z,
                int kchunk, float* ws) {
  const dim3 block(TL::THREADS);
  if constexpr (CS) {  // the launcher has checked bm == kVecMN
    hipLaunchKernelGGL((gemm_kernel<TL, AM, kVecMN, ACT, true>), grid, block, 0, st, A, B, C, ep,
                       M, N, K, zin, Z, kchunk, ws);
    return;
  }
  if (bm == kVecK)
    hipLaunchKernelGGL((gemm_kernel<TL, AM, kVecK, ACT>), grid, block, 0, st, A, B, C, ep, M, N,
                       K, zin, Z, kchunk, ws);
  else if (bm == kVecMN)
    hipLaunchKernelGGL((gemm_kernel<TL, AM, kVecMN, ACT>), grid, block, 0, st, A, B, C, ep, M, N,
                       K, zin, Z, kchunk, ws);
  else
    hipLaunchKernelGGL((gemm_kernel<TL, AM, kScalar, ACT>), grid, block, 0, st, A, B, C, ep, M,
                       N, K, zin, Z, kchunk, ws);
}

template <class TL, int ACT, bool CS = false>
void dispatch_a(int am, int bm, dim3 grid, hipStream_t st, const GemmOperand& A,
                const GemmOperand& B, const GemmOut& C, const GemmEpilogue& ep, int M, int N,
                int K, int zin, int Z, int kchunk, float* ws) {
  if (am == kVecK)
    dispatch_b<TL, kVecK, ACT, CS>(bm, grid, st, A, B, C, ep, M, N, K, zin, Z, kchunk, ws);
  else if (am == kVecMN)
    dispatch_b<TL, kVecMN, ACT, CS>(bm, grid, st, A, B, C, ep, M, N, K, zin, Z, kchunk, ws);
  else
    dispatch_b<TL, kScalar, ACT, CS>(bm, grid, st, A, B, C, ep, M, N, K, zin, Z, kchunk, ws);
}

// K splits for a GEMM whose output tiles alone cannot fill the 256 CUs (1 = no split).  The
// busiest CU runs ceil(tiles S / 256) workgroups of ceil(K / S) each, and the split adds a
// round trip of S partial outputs through HBM; S in [1, 32] (at least 256 of K per split)
// minimises the sum.  Costs are in seconds at an MFMA rate of ~0.4 TFLOP/s per CU and
// ~5 TB/s of HBM.  E.g. the 768 x 3072 x 8192 weight gradient: 144 tiles, S = 7 (1008
// workgroups, 98% of the CUs' time busy) where a plain "~512 workgroups" rule gives S = 4
// (576 workgroups, three rounds for 2.25 rounds of work); the 384 x 384 x 16384 one: 9 tiles,
// S = 28 (252 workgroups; capped at 16 it left 112 CUs idle and ran 27% slower).
template <class TL>
int64_t splitk_factor(int64_t M, int64_t N, int64_t K, int64_t Z) {
  const int64_t tiles = ((M + TL::BM - 1) / TL::BM) * ((N + TL::BN - 1) / TL::BN) * Z;
  if (tiles >= 256 || K < 1024) return 1;
  constexpr double kCuFlops = 0.4e12, kHbmBytes = 5e12;
  const double tile_flop_per_k = 2.0 * TL::BM * TL::BN;
  int64_t best = 1;
  double best_cost = 0.0;
  for (int64_t s = 1; s <= 32 && (s == 1 || K / s >= 256); ++s) {
    const int64_t kchunk = ((K + s - 1) / s + TL::BK - 1) / TL::BK * TL::BK;
    const int64_t rounds = (tiles * s + 255) / 256;
    const double cost = (double)rounds * kchunk * tile_flop_per_k / kCuFlops +
                        (s > 1 ? 8.0 * s * M * N * Z / kHbmBytes : 0.0);
    if (s == 1 || cost < best_cost) { best = s; best_cost = cost; }
  }
  return best;
}

// ACTS = false: a tile instantiated without the pointwise stages (ep.act must be kActNone).
template <class TL, bool ACTS = true>
int gemm_launch_tile(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                     const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                     int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats) {
  if (M <= 0 || N <= 0 || Z <= 0) return CTA_OK;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || Z > 65535 || zin <= 0)
    return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM size out of range");
  int64_t S = splitk_factor<TL>(M, N, K, Z);
  const int64_t cs_floats = ep.colsum ? N : 0;  // per split
  if (S > 1 && (workspace == nullptr || workspace_floats < S * (Z * M * N + cs_floats))) S = 1;
  const int64_t kchunk =
      S > 1 ? ((K + S - 1) / S + TL::BK - 1) / TL::BK * TL::BK : std::max<int64_t>(K, 1);
  const int64_t ntiles = ((N + TL::BN - 1) / TL::BN) * ((M + TL::BM - 1) / TL::BM);
  if (ntiles * Z > INT32_MAX - kNumXcds || Z * S > 65535)
    return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM grid too large");
  const dim3 grid = S > 1 ? dim3((unsigned)((N + TL::BN - 1) / TL::BN),
                                 (unsigned)((M + TL::BM - 1) / TL::BM), (unsigned)(Z * S))
                          : dim3(xcd_grid(ntiles * Z), 1, 1);
  if (grid.y > 65535) return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM grid too large");
  float* ws = S > 1 ? workspace : nullptr;
  const int am = pick_mode(A, true, M, K);
  const int bm = pick_mode(B, false, N, K);
  // Split-K partials are stored raw; the reduction applies the epilogue's pointwise stage.
  const int act = S > 1 ? kActNone : ep.act;
  const int iM = (int)M, iN = (int)N, iK = (int)K, izin = (int)zin, iZ = (int)Z, ikc = (int)kchunk;
  if (ep.colsum) {
    if (Z != 1 || bm != kVecMN || ep.act != kActNone || ep.causal_mask)
      return fail(CTA_ERR_INVALID_ARGUMENT,
                  "GEMM column sums need one batch, an n-contiguous B and no pointwise stage");
    dispatch_a<TL, kActNone, true>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
  } else if constexpr (!ACTS) {
    if (act != kActNone) return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM tile without pointwise stages");
    dispatch_a<TL, kActNone>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
  } else {
    if (act == kActGelu)
      dispatch_a<TL, kActGelu>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
    else if (act == kActGeluGrad)
      dispatch_a<TL, kActGeluGrad>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
    else if (act == kActGeluTanh)
      dispatch_a<TL, kActGeluTanh>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
    else if (act == kActGeluTanhGrad)
      dispatch_a<TL, kActGeluTanhGrad>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc,
                                       ws);
    else if (act == kActGeluDeriv)
      dispatch_a<TL, kActGeluDeriv>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
    else if (act == kActGeluTanhDeriv)
      dispatch_a<TL, kActGeluTanhDeriv>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc,
                                        ws);
    else if (act == kActMulAux)
      dispatch_a<TL, kActMulAux>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
    else
      dispatch_a<TL, kActNone>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
  }
  if (S > 1) {
    const int64_t total = Z * M * N + cs_floats;
    const unsigned rgrid = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(rgrid), dim3(256), 0, st, ws, (int)S, (int)Z,
                       (int)M, (int)N, C, ep, (int)zin);
  }
  return check_launch("gemm");
}

// Tile choice, from measured sweeps of the config-4 and small-GPT shapes on an MI355X:
// narrow outputs (N <= 768) run best with a 64x128 tile of four 32x64 waves and K-slices of 32,
// wider ones with a 128x128 tile of four 64x64 waves, and shapes split along K with a 128x128
// tile of eight 32x64 waves.  When N is a multiple of 192 the same shapes with 192 columns
// (waves of 32x96 or 64x96) measured 0-8% faster (cold, A/B in one process): 64x192 with
// K-slices of 16 for K <= 512 and of 32 beyond, and, without a pointwise stage, 128x192 with
// K-slices of 16 for N > 768 (with the GELU stages it was slower in the GPT step).
using SplitTile = GemmTile<128, 128, 16, 4, 2>;
using NarrowTile = GemmTile<64, 128, 32, 2, 2>;
using Narrow192Tile = GemmTile<64, 192, 32, 2, 2>;
using Narrow192ShortKTile = GemmTile<64, 192, 16, 2, 2>;
using WideTile = GemmTile<128, 128, 16, 2, 2>;
using Wide192Tile = GemmTile<128, 192, 16, 2, 2>;

}  // namespace

// One launcher per tile type (defined in gemm_tiles_*.hip): gemm_launch_tile of that tile.
int gemm_launch_split(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                      const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                      int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats);
int gemm_launch_narrow(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                       const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                       int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats);
int gemm_launch_narrow192(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                          const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                          int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats);
int gemm_launch_narrow192_short_k(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                                  const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                                  int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats);
int gemm_launch_wide(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                     const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                     int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats);
int gemm_launch_wide192(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                        const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                        int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats);

}  // namespace cta
