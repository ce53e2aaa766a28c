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
// gfx950 design: workgroup tile 128x128 of eight 32x64 waves (4x2) or 128x64 of four 64x32
// waves, each wave owning a block of v_mfma_f32_32x32x2_f32 tiles.  A and B tiles are staged
// through LDS as [m][k] and [n][k] (k contiguous, pitch BK+4), so each MFMA operand fragment is a pair of
// conflict-free 16-byte LDS reads whatever the operand's memory order.  Global loads are
// dwordx4 along whichever dimension is contiguous in memory (template mode), with scalar
// loads for ragged edges and irregular strides.  Within a slice the instruction order is pinned
// (sched_group_barrier): global loads and LDS stores sit between the MFMAs, and the next
// slice's fragments are read while the current slice's last MFMAs run.
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
template <int MODE, int ROWS, int BK, int THREADS>
struct TileLoader {
  static constexpr int LOADS = ROWS * BK / 4 / THREADS;
  static_assert(ROWS * BK % (4 * THREADS) == 0, "tile must split evenly over the workgroup");
  float4 v[LOADS];
  bool kin[LOADS];  // vector modes: the float4 lies inside K (zeroed at store time otherwise)
  __device__ __forceinline__ void load(const float* base, int64_t s_row, int64_t s_k, int row0,
                                       int k0, int R, int K, int tid) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + THREADS * u;
      if (MODE == kVecMN) {
        // k varies fastest across lanes: each 16-lane group reads 64 contiguous bytes of one k
        // row and the LDS transpose below writes 16 consecutive words (no bank conflicts).
        // Branch-free: always one dwordx4 from a clamped in-bounds address (R % 4 == 0), so the
        // wait counters stay exact.  Rows past R only feed output rows/columns that are never
        // stored; k past K must contribute zero and is masked when the slice is stored to LDS.
        const int k = f % BK, r4 = (f / BK) * 4;
        const int gr = row0 + r4, gk = k0 + k;
        v[u] = ld4(base + (int64_t)min(gk, K - 1) * s_k + min(gr, R - 4));
        kin[u] = gk < K;
      } else if (MODE == kVecK) {
        int r, k4;
        veck_coords<BK>(f, r, k4);
        const int gr = row0 + r, gk = k0 + k4;
        v[u] = ld4(base + (int64_t)min(gr, R - 1) * s_row + min(gk, K - 4));
        kin[u] = gk < K;  // K % 4 == 0: a float4 is wholly inside or outside
      } else {
        int r, k4;
        veck_coords<BK>(f, r, k4);
        const int gr = row0 + r, gk = k0 + k4;
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          t[e] = (gr < R && gk + e < K) ? base[(int64_t)gr * s_row + (int64_t)(gk + e) * s_k] : 0.0f;
        v[u] = make_float4(t[0], t[1], t[2], t[3]);
        kin[u] = true;
      }
    }
  }
  // LDS image: [row][k], pitch BK + 4.
  __device__ __forceinline__ void store(float* lds, int tid) const {
    constexpr int KP = BK + 4;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int f = tid + THREADS * u;
      const float4 w = kin[u] ? v[u] : zero4();
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
};

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

// The epilogue of one output tile (origin m0, n0 of batch (zo, zi)): alpha, bias, causal mask
// and the pointwise stage ACT, stored through C.
template <class TL, int ACT>
__device__ __forceinline__ void tile_store(const f32x16 (&acc)[TL::MB][TL::NB], const GemmOut& C,
                                           const GemmEpilogue& ep, int M, int N, int m0, int n0,
                                           int zo, int zi, int wm, int wn, int half, int col) {
  constexpr int BM = TL::BM, BN = TL::BN, MB = TL::MB, NB = TL::NB;
  float* Cb = C.p + zo * C.s_outer + zi * C.s_inner;
  float* Xb = ep.aux ? ep.aux + zo * C.s_outer + zi * C.s_inner : nullptr;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = n0 + wn * (BN / TL::WN) + j * 32 + col;
    if (n >= N) continue;
    const float bv = ep.bias ? ep.bias[(int64_t)n * ep.bias_stride] : 0.0f;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm * (BM / TL::WM) + i * 32 + mfma_row(r, half);
        if (m < M) {
          float val = fmaf(ep.alpha, acc[i][j][r], bv);
          if (ep.causal_mask && n > m) val = -INFINITY;
          const int64_t off = (int64_t)m * C.s_row + n;
          if (ACT == kActGeluGrad) val = gelu_grad(Xb[off], val);
          if (ACT == kActGeluTanhGrad) val = gelu_tanh_grad(Xb[off], val);
          Cb[off] = val;
          if (ACT == kActGelu) Xb[off] = gelu_f(val);
          if (ACT == kActGeluTanh) Xb[off] = gelu_tanh_f(val);
        }
      }
    }
  }
}

// split_ws == nullptr: out = alpha * A B (+ bias, mask) written through C.
// split_ws != nullptr: blockIdx.z = s * Z + z covers K range [s*kchunk, (s+1)*kchunk) and the raw
// partial sum goes to split_ws[s][z][m][n] (dense); gemm_splitk_reduce finishes the epilogue.
template <class TL, int AMODE, int BMODE, int ACT>
__global__ __launch_bounds__(TL::THREADS) void gemm_kernel(GemmOperand A, GemmOperand B,
                                                           GemmOut C, GemmEpilogue ep, int M,
                                                           int N, int K, int zin, int Z,
                                                           int kchunk,
                                                           float* __restrict__ split_ws) {
  constexpr int BM = TL::BM, BN = TL::BN, BK = TL::BK, KP = TL::KP;
  constexpr int MB = TL::MB, NB = TL::NB;
  __shared__ __attribute__((aligned(16))) float smem[TL::LDS_FLOATS];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, col = lane & 31;
  const int wm = wave / TL::WN, wn = wave % TL::WN;

  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int z = blockIdx.z % Z, split = blockIdx.z / Z;
  const int zo = z / zin, zi = z - zo * zin;
  const float* Ab = A.p + zo * A.s_outer + zi * A.s_inner;
  const float* Bb = B.p + zo * B.s_outer + zi * B.s_inner;
  const int kb = split * kchunk;
  const int ke = min(K, kb + kchunk);

  // A rows are m with (s_row, s_col) = (m, k); B "rows" are n with (n, k) = (s_col, s_row).
  // Global loads run two K-slices ahead of the MFMAs (two register sets, alternating), so a
  // slice's loads have two slices of MFMA work to arrive; LDS is double buffered.  Vector-mode
  // loads clamp their addresses into the operand, so reads past K stay in bounds.
  using LA = TileLoader<AMODE, BM, BK, TL::THREADS>;
  using LB = TileLoader<BMODE, BN, BK, TL::THREADS>;
  LA la0, la1;
  LB lb0, lb1;
  const int nk = (ke - kb + BK - 1) / BK;

  f32x16 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = zero16();

  // Slice count rounded up to even: slices past the end load clamped addresses whose k lies
  // beyond ke, so they are stored as zeros and add nothing.  The loop then has no conditional
  // loads or stores, which keeps the compiler's wait counts exact (a load issued two slices
  // ahead is not waited for until its LDS store).
  const int nk2 = (nk + 1) & ~1;
  la0.load(Ab, A.s_row, A.s_col, m0, kb, M, ke, tid);
  lb0.load(Bb, B.s_col, B.s_row, n0, kb, N, ke, tid);
  la1.load(Ab, A.s_row, A.s_col, m0, kb + BK, M, ke, tid);
  lb1.load(Bb, B.s_col, B.s_row, n0, kb + BK, N, ke, tid);
  la0.store(smem, tid);
  lb0.store(smem + BM * KP, tid);
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
    la0.load(Ab, A.s_row, A.s_col, m0, kb + (t + 2) * BK, M, ke, tid);
    lb0.load(Bb, B.s_col, B.s_row, n0, kb + (t + 2) * BK, N, ke, tid);
    mma_chunks<TL, 0, KC / 2>(f0, acc);
    la1.store(buf1, tid);
    lb1.store(buf1 + BM * KP, tid);
    sched_first_part<0, NM1, NVM, NDW>();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_frags<TL>(buf1, f1, wm, wn, half, col);
    mma_chunks<TL, KC / 2, KC>(f0, acc);
    __builtin_amdgcn_sched_group_barrier(0x100, NDR, 0);  // LDS reads first
    __builtin_amdgcn_sched_group_barrier(0x008, NM1, 0);
    __builtin_amdgcn_sched_barrier(0);
    // slice t+1 in f1
    la1.load(Ab, A.s_row, A.s_col, m0, kb + (t + 3) * BK, M, ke, tid);
    lb1.load(Bb, B.s_col, B.s_row, n0, kb + (t + 3) * BK, N, ke, tid);
    mma_chunks<TL, 0, KC / 2>(f1, acc);
    la0.store(buf0, tid);
    lb0.store(buf0 + BM * KP, tid);
    sched_first_part<0, NM1, NVM, NDW>();
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_frags<TL>(buf0, f0, wm, wn, half, col);
    mma_chunks<TL, KC / 2, KC>(f1, acc);
    __builtin_amdgcn_sched_group_barrier(0x100, NDR, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, NM1, 0);
    __builtin_amdgcn_sched_barrier(0);
  }

  if (split_ws != nullptr) {
    float* Pb = split_ws + ((int64_t)split * Z + z) * M * N;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = n0 + wn * (BN / TL::WN) + j * 32 + col;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm * (BM / TL::WM) + i * 32 + mfma_row(r, half);
          if (m < M) Pb[(int64_t)m * N + n] = acc[i][j][r];
        }
    }
    return;
  }
  tile_store<TL, ACT>(acc, C, ep, M, N, m0, n0, zo, zi, wm, wn, half, col);
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
    const int64_t off = zo * C.s_outer + zi * C.s_inner + (int64_t)m * C.s_row + n;
    if (ep.act == kActGeluGrad) val = gelu_grad(ep.aux[off], val);
    if (ep.act == kActGeluTanhGrad) val = gelu_tanh_grad(ep.aux[off], val);
    C.p[off] = val;
    if (ep.act == kActGelu) ep.aux[off] = gelu_f(val);
    if (ep.act == kActGeluTanh) ep.aux[off] = gelu_tanh_f(val);
  }
}

bool vec_ok(const GemmOperand& op, bool contig_is_col) {
  // dwordx4 loads along the contiguous dimension need 16-byte aligned rows.
  const int64_t s_other = contig_is_col ? op.s_row : op.s_col;
  return aligned16(op.p) && s_other % 4 == 0 && op.s_outer % 4 == 0 && op.s_inner % 4 == 0;
}

// Load mode of an operand.  A: (s_row, s_col) = (m, k); B: (k, n).  `rows` is M for A and N for
// B.  The vector modes also need the contiguous extent to be a multiple of 4 (the branch-free
// loads clamp whole float4s) and at least 4.
int pick_mode(const GemmOperand& op, bool is_a, int64_t rows, int64_t K) {
  const int64_t s_k = is_a ? op.s_col : op.s_row;
  const int64_t s_mn = is_a ? op.s_row : op.s_col;
  if (s_k == 1 && K % 4 == 0 && K >= 4 && vec_ok(op, is_a)) return kVecK;
  if (s_mn == 1 && rows % 4 == 0 && rows >= 4 && vec_ok(op, !is_a)) return kVecMN;
  return kScalar;
}

template <class TL, int AM, int ACT>
void dispatch_b(int bm, dim3 grid, hipStream_t st, const GemmOperand& A, const GemmOperand& B,
                const GemmOut& C, const GemmEpilogue& ep, int M, int N, int K, int zin, int Z,
                int kchunk, float* ws) {
  const dim3 block(TL::THREADS);
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

template <class TL, int ACT>
void dispatch_a(int am, int bm, dim3 grid, hipStream_t st, const GemmOperand& A,
                const GemmOperand& B, const GemmOut& C, const GemmEpilogue& ep, int M, int N,
                int K, int zin, int Z, int kchunk, float* ws) {
  if (am == kVecK)
    dispatch_b<TL, kVecK, ACT>(bm, grid, st, A, B, C, ep, M, N, K, zin, Z, kchunk, ws);
  else if (am == kVecMN)
    dispatch_b<TL, kVecMN, ACT>(bm, grid, st, A, B, C, ep, M, N, K, zin, Z, kchunk, ws);
  else
    dispatch_b<TL, kScalar, ACT>(bm, grid, st, A, B, C, ep, M, N, K, zin, Z, kchunk, ws);
}

// K splits for a GEMM whose output tiles alone cannot fill the 256 CUs (1 = no split).  The
// busiest CU runs ceil(tiles S / 256) workgroups of ceil(K / S) each, and the split adds a
// round trip of S partial outputs through HBM; S in [1, 16] (at least 256 of K per split)
// minimises the sum.  Costs are in seconds at an MFMA rate of ~0.4 TFLOP/s per CU and
// ~5 TB/s of HBM.  E.g. the 768 x 3072 x 8192 weight gradient: 144 tiles, S = 7 (1008
// workgroups, 98% of the CUs' time busy) where a plain "~512 workgroups" rule gives S = 4
// (576 workgroups, three rounds for 2.25 rounds of work).
template <class TL>
int64_t splitk_factor(int64_t M, int64_t N, int64_t K, int64_t Z) {
  const int64_t tiles = ((M + TL::BM - 1) / TL::BM) * ((N + TL::BN - 1) / TL::BN) * Z;
  if (tiles >= 256 || K < 1024) return 1;
  constexpr double kCuFlops = 0.4e12, kHbmBytes = 5e12;
  const double tile_flop_per_k = 2.0 * TL::BM * TL::BN;
  int64_t best = 1;
  double best_cost = 0.0;
  for (int64_t s = 1; s <= 16 && (s == 1 || K / s >= 256); ++s) {
    const int64_t kchunk = ((K + s - 1) / s + TL::BK - 1) / TL::BK * TL::BK;
    const int64_t rounds = (tiles * s + 255) / 256;
    const double cost = (double)rounds * kchunk * tile_flop_per_k / kCuFlops +
                        (s > 1 ? 8.0 * s * M * N * Z / kHbmBytes : 0.0);
    if (s == 1 || cost < best_cost) { best = s; best_cost = cost; }
  }
  return best;
}

template <class TL>
int gemm_launch_tile(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                     const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z,
                     int64_t zin, hipStream_t st, float* workspace, int64_t workspace_floats) {
  if (M <= 0 || N <= 0 || Z <= 0) return CTA_OK;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || Z > 65535 || zin <= 0)
    return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM size out of range");
  int64_t S = splitk_factor<TL>(M, N, K, Z);
  if (S > 1 && (workspace == nullptr || workspace_floats < S * Z * M * N)) S = 1;
  const int64_t kchunk =
      S > 1 ? ((K + S - 1) / S + TL::BK - 1) / TL::BK * TL::BK : std::max<int64_t>(K, 1);
  const dim3 grid((unsigned)((N + TL::BN - 1) / TL::BN), (unsigned)((M + TL::BM - 1) / TL::BM),
                  (unsigned)(Z * S));
  if (grid.y > 65535 || grid.z > 65535) return fail(CTA_ERR_INVALID_ARGUMENT, "GEMM grid too large");
  float* ws = S > 1 ? workspace : nullptr;
  const int am = pick_mode(A, true, M, K);
  const int bm = pick_mode(B, false, N, K);
  // Split-K partials are stored raw; the reduction applies the epilogue's pointwise stage.
  const int act = S > 1 ? kActNone : ep.act;
  const int iM = (int)M, iN = (int)N, iK = (int)K, izin = (int)zin, iZ = (int)Z, ikc = (int)kchunk;
  if (act == kActGelu)
    dispatch_a<TL, kActGelu>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
  else if (act == kActGeluGrad)
    dispatch_a<TL, kActGeluGrad>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
  else if (act == kActGeluTanh)
    dispatch_a<TL, kActGeluTanh>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
  else if (act == kActGeluTanhGrad)
    dispatch_a<TL, kActGeluTanhGrad>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc,
                                     ws);
  else
    dispatch_a<TL, kActNone>(am, bm, grid, st, A, B, C, ep, iM, iN, iK, izin, iZ, ikc, ws);
  if (S > 1) {
    const int64_t total = Z * M * N;
    const unsigned rgrid = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    hipLaunchKernelGGL(gemm_splitk_reduce, dim3(rgrid), dim3(256), 0, st, ws, (int)S, (int)Z,
                       (int)M, (int)N, C, ep, (int)zin);
  }
  return check_launch("gemm");
}

// Tile choice, from measured sweeps of the config-4 and small-GPT shapes on an MI355X:
// narrow outputs (N <= 768) run best with a 128x64 tile of four 64x32 waves, everything else
// (including shapes split along K) with a 128x128 tile of eight 32x64 waves.
using SplitTile = GemmTile<128, 128, 16, 4, 2>;
using NarrowTile = GemmTile<128, 64, 16, 2, 2>;
using WideTile = GemmTile<128, 128, 16, 4, 2>;

}  // namespace

int64_t gemm_workspace_floats(int64_t M, int64_t N, int64_t K, int64_t Z) {
  const int64_t S = splitk_factor<SplitTile>(M, N, K, Z);
  return S > 1 ? S * Z * M * N : 0;
}

// Launch the strided batched GEMM.  Z = number of batches, zin = inner batch extent.  With a
// workspace of gemm_workspace_floats() floats, low-parallelism shapes are split along K.
int gemm_launch(const GemmOperand& A, const GemmOperand& B, const GemmOut& C,
                const GemmEpilogue& ep, int64_t M, int64_t N, int64_t K, int64_t Z, int64_t zin,
                hipStream_t st, float* workspace, int64_t workspace_floats) {
  const int64_t S = splitk_factor<SplitTile>(M, N, K, Z);
  if (S > 1 && workspace != nullptr && workspace_floats >= S * Z * M * N)
    return gemm_launch_tile<SplitTile>(A, B, C, ep, M, N, K, Z, zin, st, workspace,
                                       workspace_floats);
  if (N <= 768)
    return gemm_launch_tile<NarrowTile>(A, B, C, ep, M, N, K, Z, zin, st, nullptr, 0);
  return gemm_launch_tile<WideTile>(A, B, C, ep, M, N, K, Z, zin, st, nullptr, 0);
}

}  // namespace cta

using namespace cta;

extern "C" int64_t cta_cuda_fma_workspace(int64_t batch, int64_t m, int64_t k, int64_t n) {
  if (batch <= 0 || m <= 0 || n <= 0 || k <= 0) return 0;
  return gemm_workspace_floats(m, n, k, batch) * (int64_t)sizeof(float);
}

namespace {
// out[b] = x[b] . W[b or 0] with epilogue `ep`, out dense (batch, m, n): the shared body of the
// linear-layer entry points.  Weights broadcast over the batch with batch stride 0 when
// w_batch == 1, as linear_layer.cu:30-34 does.
int linear_launch(const float* x, const int64_t* x_strides, const float* w,
                  const int64_t* w_strides, int64_t batch, int64_t m, int64_t k, int64_t n,
                  int64_t w_batch, float* out, const GemmEpilogue& ep, float* workspace,
                  void* stream) {
  if (batch < 0 || m < 0 || k < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (w_batch != 1 && w_batch != batch)
    return fail(CTA_ERR_INVALID_ARGUMENT, "weights batch must be 1 or equal to x batch");
  if (batch * m * n == 0) return CTA_OK;
  if (!x || !w || !out || !x_strides || !w_strides)
    return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  const GemmOperand A{x, x_strides[0], 0, x_strides[1], x_strides[2]};
  const GemmOperand B{w, w_batch == 1 ? 0 : w_strides[0], 0, w_strides[1], w_strides[2]};
  const GemmOut C{out, m * n, 0, n};
  return gemm_launch(A, B, C, ep, m, n, k, batch, 1, as_stream(stream), workspace,
                     workspace ? gemm_workspace_floats(m, n, k, batch) : 0);
}
}  // namespace

extern "C" int cta_cuda_fma(const float* x, const int64_t* x_strides, const float* w,
                            const int64_t* w_strides, const float* bias, int64_t bias_stride,
                            int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                            float* out, float* workspace, void* stream) {
  if (!bias && batch > 0 && m > 0 && n > 0) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  const GemmEpilogue ep{1.0f, bias, bias_stride, 0};
  return linear_launch(x, x_strides, w, w_strides, batch, m, k, n, w_batch, out, ep, workspace,
                       stream);
}

namespace {
int fma_act(const float* x, const int64_t* x_strides, const float* w, const int64_t* w_strides,
            const float* bias, int64_t bias_stride, int64_t batch, int64_t m, int64_t k,
            int64_t n, int64_t w_batch, float* pre, float* out, float* workspace, void* stream,
            int act) {
  if (batch > 0 && m > 0 && n > 0) {
    if (!bias || !out) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
    if (pre == out) return fail(CTA_ERR_INVALID_ARGUMENT, "pre and out must be distinct buffers");
  }
  const GemmEpilogue ep{1.0f, bias, bias_stride, 0, act, out};
  return linear_launch(x, x_strides, w, w_strides, batch, m, k, n, w_batch, pre, ep, workspace,
                       stream);
}

int fma_act_grad(const float* dy, const int64_t* dy_strides, const float* w,
                 const int64_t* w_strides, const float* pre, int64_t batch, int64_t m, int64_t k,
                 int64_t n, int64_t w_batch, float* dx, float* workspace, void* stream, int act) {
  if (!pre && batch > 0 && m > 0 && n > 0) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  // Each output element reads its own pre-activation just before it is stored, so dx may
  // alias pre.
  const GemmEpilogue ep{1.0f, nullptr, 0, 0, act, const_cast<float*>(pre)};
  return linear_launch(dy, dy_strides, w, w_strides, batch, m, k, n, w_batch, dx, ep, workspace,
                       stream);
}
}  // namespace

extern "C" int cta_cuda_fma_gelu(const float* x, const int64_t* x_strides, const float* w,
                                 const int64_t* w_strides, const float* bias,
                                 int64_t bias_stride, int64_t batch, int64_t m, int64_t k,
                                 int64_t n, int64_t w_batch, float* pre, float* out,
                                 float* workspace, void* stream) {
  return fma_act(x, x_strides, w, w_strides, bias, bias_stride, batch, m, k, n, w_batch, pre, out,
                 workspace, stream, kActGelu);
}

extern "C" int cta_cuda_fma_gelu_grad(const float* dy, const int64_t* dy_strides, const float* w,
                                      const int64_t* w_strides, const float* pre, int64_t batch,
                                      int64_t m, int64_t k, int64_t n, int64_t w_batch,
                                      float* dx, float* workspace, void* stream) {
  return fma_act_grad(dy, dy_strides, w, w_strides, pre, batch, m, k, n, w_batch, dx, workspace,
                      stream, kActGeluGrad);
}

extern "C" int cta_cuda_fma_gelu_tanh(const float* x, const int64_t* x_strides, const float* w,
                                      const int64_t* w_strides, const float* bias,
                                      int64_t bias_stride, int64_t batch, int64_t m, int64_t k,
                                      int64_t n, int64_t w_batch, float* pre, float* out,
                                      float* workspace, void* stream) {
  return fma_act(x, x_strides, w, w_strides, bias, bias_stride, batch, m, k, n, w_batch, pre, out,
                 workspace, stream, kActGeluTanh);
}

extern "C" int cta_cuda_fma_gelu_tanh_grad(const float* dy, const int64_t* dy_strides,
                                           const float* w, const int64_t* w_strides,
                                           const float* pre, int64_t batch, int64_t m, int64_t k,
                                           int64_t n, int64_t w_batch, float* dx,
                                           float* workspace, void* stream) {
  return fma_act_grad(dy, dy_strides, w, w_strides, pre, batch, m, k, n, w_batch, dx, workspace,
                      stream, kActGeluTanhGrad);
}

extern "C" int64_t cta_db_calculation_workspace(int64_t batch, int64_t m, int64_t n) {
  if (batch <= 0 || m <= 0 || n <= 0) return 0;
  return colsum_workspace_floats(batch * m, n) * (int64_t)sizeof(float);
}

extern "C" int cta_db_calculation(const float* dy, const int64_t* dy_strides, int64_t batch,
                                  int64_t m, int64_t n, float* db, float* workspace,
                                  void* stream) {
  if (batch < 0 || m < 0 || n < 0) return fail(CTA_ERR_INVALID_ARGUMENT, "negative size");
  if (n == 0) return CTA_OK;
  if (!db) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  hipStream_t st = as_stream(stream);
  if (batch * m == 0) return zero_floats(db, n, st);
  if (!dy || !dy_strides || !workspace) return fail(CTA_ERR_INVALID_ARGUMENT, "null pointer");
  return colsum_launch(dy, batch, m, n, dy_strides[0], dy_strides[1], dy_strides[2], db,
                       workspace, st);
}
