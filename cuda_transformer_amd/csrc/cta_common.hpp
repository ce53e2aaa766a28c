// Shared device helpers and host-side error plumbing for the gfx950 kernels.
//
// Every kernel in this library is written for CDNA4 (gfx950): wave64, FP32 MFMA
// (v_mfma_f32_32x32x2_f32), LDS tiles with padded pitches.  The lane layout of the
// 32x32x2 MFMA that all attention / GEMM kernels rely on (checked on an MI355X):
//   A operand (32 x 2):  lane l supplies A[l % 32][l / 32]
//   B operand (2 x 32):  lane l supplies B[l / 32][l % 32]
//   D (32 x 32, 16 regs): lane l, register r holds D[R(r, l/32)][l % 32]
//                         with R(r, h) = 8*(r/4) + 4*h + (r%4)
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <algorithm>
#include <cmath>
#include <string>

#include "../../include/cuda_transformer_amd.h"

namespace cta {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16 bytes of 16-bit elements

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Row index inside a 32x32 MFMA output tile held by register r of a lane in half h.
__device__ __forceinline__ constexpr int mfma_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// Streaming (non-temporal) 16-byte load and store, for data touched once per pass whose total
// far exceeds the caches (the stored dS tiles): the access carries the `nt` bit, so it does not
// displace the reused K/V/Q rows from L2.
typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld4_stream(const float* p) {
  const nt_f32x4 x = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4*>(p));
  return make_float4(x[0], x[1], x[2], x[3]);
}
__device__ __forceinline__ void st4_stream(float* p, float4 v) {
  const nt_f32x4 x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<nt_f32x4*>(p));
}

// 16-bit MFMA (gfx950 v_mfma_f32_32x32x16_bf16 / _f16), checked on an MI355X for BF16 and
// shared by the FP16 form:
//   A (32 x 16): lane l supplies A[l % 32][8 (l/32) + j], j = 0..7
//   B (16 x 32): lane l supplies B[8 (l/32) + j][l % 32]
//   D: the 32x32 layout of the FP32 MFMA above.
// Half16<E> carries the 8-element operand type and the MFMA for E = __bf16 or _Float16.
template <class E>
struct Half16;
template <>
struct Half16<__bf16> {
  typedef __bf16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Half16<_Float16> {
  typedef _Float16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mfma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <class E>
using vec8_t = typename Half16<E>::vec8;
template <class E>
__device__ __forceinline__ vec8_t<E> ld8(const E* p) {
  return *reinterpret_cast<const vec8_t<E>*>(p);
}
// Streaming forms of the 16-byte 16-bit vector access, for the stored dS tiles.
template <class E>
__device__ __forceinline__ vec8_t<E> ld8_stream(const E* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const vec8_t<E>*>(p));
}
template <class E>
__device__ __forceinline__ void st8_stream(E* p, vec8_t<E> v) {
  __builtin_nontemporal_store(v, reinterpret_cast<vec8_t<E>*>(p));
}
// A 32x32 score tile in registers (lane l: rows R(r, l/32)) is the B operand of two 16-deep
// BF16 MFMA steps: step s takes registers 8s .. 8s+7, i.e. rows 16 s + 8 (j/4) + 4 h + j%4 of
// element j.  A matching A operand read from a transposed [col][row] image in LDS needs those
// rows adjacent: store row k of the image at position kt_pos(k), bits 2 and 3 of k swapped.
__device__ __forceinline__ constexpr int kt_pos(int k) {
  return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

// Interleave the 16-bit halves of two words with one v_perm_b32: pack_lo16(a, b) holds the low
// halves (a's in bits 0-15, b's in bits 16-31), pack_hi16(a, b) the high halves.
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// Index of this thread's wave in a 256-thread workgroup, marked wave-uniform for the compiler
// (through readfirstlane), so that branches on it are scalar branches.
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Maximum of v[0 .. N) as a tree of three-input maxima, depth log3(N): the form v_max3_f32
// implements.  Overwrites v.
template <int N>
__device__ __forceinline__ float max3_tree(float (&v)[N]) {
  constexpr int M = (N + 2) / 3;
  float w[M];
#pragma unroll
  for (int k = 0; k < M; ++k) {
    float a = v[3 * k];
    if (3 * k + 1 < N) a = fmaxf(a, v[3 * k + 1]);
    if (3 * k + 2 < N) a = fmaxf(a, v[3 * k + 2]);
    w[k] = a;
  }
  if constexpr (M == 1) return w[0];
  else return max3_tree(w);
}

// Exchange with the lane 32 positions away (the other half of the wave).
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32); }

// Combine the two wave halves with v_permlane32_swap (gfx950): a VALU lane swap with no LDS
// round trip.  Swapping a register with itself leaves r[0] = v of lane (l % 32) and
// r[1] = v of lane (l % 32) + 32 in every lane, so both halves compute the same operands in
// the same order and get bitwise identical results.
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// MI355X dispatches workgroup ids round-robin over its 8 XCDs, each with a private 4 MB L2.
// Remap the hardware id so that XCD x walks the contiguous run [x*per, (x+1)*per) of a
// work list: when that list is ordered head-major, the workgroups resident on one XCD share
// one or two heads' K/V instead of sixteen.  Launch 8*per workgroups; ids mapped past
// `total` have no work and exit.
constexpr int kNumXcds = 8;
__device__ __forceinline__ int xcd_work_item(int hw_id, int total) {
  const int per = (total + kNumXcds - 1) / kNumXcds;
  return (hw_id % kNumXcds) * per + hw_id / kNumXcds;
}
inline unsigned xcd_grid(int64_t total) {
  return (unsigned)(kNumXcds * ((total + kNumXcds - 1) / kNumXcds));
}

// Causal attention tiles cost unequal amounts (a query tile's keys, or a key tile's queries,
// grow along the diagonal).  The kernels pair tile p with tile n-1-p so every work item costs
// the same, or, where lpt_heads() says so, run single tiles longest first per XCD: XCD x takes
// heads [x h, (x+1) h) (h = lpt_heads) and walks their tiles tile-major, head-minor, so rank 0
// (the longest tile) of each of its heads comes first.  Grid = BH * n_tiles workgroups.
__device__ __forceinline__ void lpt_tile(int hw_id, int heads_per_xcd, int& bh, int& rank) {
  const int x = hw_id % kNumXcds, slot = hw_id / kNumXcds;
  rank = slot / heads_per_xcd;
  bh = x * heads_per_xcd + (slot - rank * heads_per_xcd);
}

// Heads per XCD for longest-first tiles, or 0 for pairs.  A grid of fewer pairs than resident
// slots leaves SIMDs at one wave; when all of an XCD's single tiles fit its resident slots at
// once, with two-wave workgroups or at most one tile per CU, they start together (so a head's
// tiles still walk its K/V stages in step and share them in L2) and the makespan is the
// longest tile, n units, against n + 1 for a pair, with more SIMDs busy.  Larger grids keep
// the pairs: longest-first tiles there measured 1-2% faster in short bursts, but the tiles that
// the dispatcher starts one by one no longer share K/V stages (L2 misses 3-4x: forward 0.65 ->
// 2.9 GB at B4 H32 N4096), and under sustained load, which holds the chip at its power limit,
// the gain was gone.  With several four-wave tiles on one CU the unequal tiles that share it
// cost more than a pair.  `waves` per workgroup, `occ` waves per SIMD the kernel holds; BH must
// split evenly over the XCDs.
constexpr int kNumSimds = 1024;
inline int lpt_heads(int64_t BH, int n_tiles, int waves, int occ) {
  if (BH % kNumXcds != 0 || n_tiles < 2) return 0;
  const int64_t tiles = BH / kNumXcds * n_tiles;                       // per XCD
  const int64_t slots = (int64_t)occ * (kNumSimds / kNumXcds) / waves;  // resident per XCD
  const int64_t cus = kNumSimds / kNumXcds / 4;
  return tiles <= slots && (waves == 2 || tiles <= cus) ? (int)(BH / kNumXcds) : 0;
}

// Stored dS tiles of the backward (FA2, FP32 and BF16).  Tile (ib, jb) covers query rows
// 32*ib.. and key rows 32*jb.. of one head; causal heads keep the tiles with jb <= ib only,
// packed row by row.
__host__ __device__ inline int64_t ds_tile_index(int ib, int jb, int nb, bool causal) {
  return causal ? (int64_t)ib * (ib + 1) / 2 + jb : (int64_t)ib * nb + jb;
}
__host__ __device__ inline int64_t ds_tiles_per_head(int64_t T, bool causal) {
  const int64_t nb = (T + 31) / 32;
  return causal ? nb * (nb + 1) / 2 : nb * nb;
}

// Asynchronous copy global -> LDS without registers (global_load_lds_dwordx4 / _dword on
// gfx950): lane l's 16 (4) bytes land at lds + 16*l (4*l), so `lds` must be the same for the
// whole wave and the wave's 64 lanes fill 1 KiB (256 B) of LDS contiguously.  Completion is
// counted by vmcnt: vm_wait_all() before the barrier that publishes the data.
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void async_copy16(const float* g, float* lds) {
  __builtin_amdgcn_global_load_lds(static_cast<const void*>(g), (lds_void_t*)(lds), 16, 0, 0);
}
__device__ __forceinline__ void async_copy4(const float* g, float* lds) {
  __builtin_amdgcn_global_load_lds(static_cast<const void*>(g), (lds_void_t*)(lds), 4, 0, 0);
}
// Buffer resource over `rows` rows (stride st floats, `width` floats used) from base; no rows:
// an empty range.  Offsets past the range read as zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float* base, int rows,
                                                            int64_t st, int width) {
  const int nbytes = rows > 0 ? (int)(((int64_t)(rows - 1) * st + width) * 4) : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, nbytes,
                                           0x00020000);
}
// The same over rows of 16-bit elements (stride st and width in elements).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc16(const void* base, int rows,
                                                              int64_t st, int width) {
  const int nbytes = rows > 0 ? (int)(((int64_t)(rows - 1) * st + width) * 2) : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nbytes,
                                           0x00020000);
}
// 16 raw bytes at byte offset voff of a buffer resource (zeros out of range).
__device__ __forceinline__ u32x4 ld16_buffer(__amdgpu_buffer_rsrc_t rs, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, 0);
}
// 16 bytes at byte offset voff of a buffer resource (zeros out of range).
__device__ __forceinline__ float4 ld4_buffer(__amdgpu_buffer_rsrc_t rs, int voff) {
  const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, 0);
  return make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z),
                     __uint_as_float(w.w));
}
// The same 16-byte copy through a buffer resource: voff is the lane's byte offset in it
// (out of range: nothing read).
__device__ __forceinline__ void async_copy16_buffer(__amdgpu_buffer_rsrc_t rs, int voff,
                                                    float* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(lds), 16, voff, 0, 0, 0);
}
// s_waitcnt vmcnt(0): all of this wave's vector memory operations have completed.
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Orders one wave's LDS accesses around a cross-lane exchange through LDS.  The hardware
// executes a wave's LDS instructions in order; the fence keeps the compiler from moving
// them across this point.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// 2^x on the hardware transcendental unit (v_exp_f32). Inputs here are <= 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Exact (erf) GELU as Transformer_kernels/GeLU.cuh:7-29 defines it: y = x Phi(x) and
// dx = dy (Phi(x) + x phi(x)), phi(x) = e^{-x^2/2} / sqrt(2 pi).
//
// Phi(x) = erfc(-x / sqrt 2) / 2, with erfc from the Chebyshev fit of Numerical Recipes
// (Press et al., 2nd ed., section 6.2, "erfcc"): for z >= 0, erfc(z) = t e^{-z^2 + r(t)} with
// t = 1 / (1 + z/2) and r a degree-9 polynomial in t, fractional error below 1.2e-7 for every
// z.  Evaluated in FP32 with the hardware reciprocal and exp2, Phi, GELU and GELU' stay within
// 4e-7 of the exact values over [-12, 12] (checked against float64 erfc).  That is about 20
// VALU instructions per element where the library normcdff took about 60, which left the
// GELU kernels VALU-bound rather than HBM-bound.
//
// The standalone GELU kernels and the GEMM epilogue share these functions (every multiply-add
// written as an explicit fmaf), so a fused linear+GELU gives the same bits as the two ops run
// one after the other.
constexpr float kInvSqrt2Pi = 0.3989422804014327f;
__device__ __forceinline__ float normal_cdf(float x) {
  const float z = fabsf(x) * 0.70710678f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(p, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  const float y = fmaf(-z, z, fmaf(p, t, -1.26551223f));  // -z^2 + r(t)
  const float h = 0.5f * t * __builtin_amdgcn_exp2f(y * kLog2e);  // erfc(z) / 2 = Phi(-|x|)
  return x < 0.0f ? h : 1.0f - h;
}
__device__ __forceinline__ float gelu_f(float x) { return x * normal_cdf(x); }
__device__ __forceinline__ float gelu_grad(float x, float g) {
  const float pdf = kInvSqrt2Pi * __builtin_amdgcn_exp2f(x * (-0.5f * kLog2e) * x);
  return g * fmaf(x, pdf, normal_cdf(x));
}

// tanh-approximated GELU, torch's F.gelu(x, approximate="tanh") (the GPT-2 form; the reference
// has no kernel for it): y = x (1 + tanh u) / 2 with u = sqrt(2/pi) (x + 0.044715 x^3).
// With a = e^{-2|u|} in (0, 1] and r = 1 / (1 + a), (1 + tanh u) / 2 is r for u >= 0 and a r
// for u < 0 (u has the sign of x), and (1 - tanh^2 u) / 4 = a r^2.  Neither form overflows or
// cancels, for any x:  y = x s  and  dy/dx = s + 2 x u' a r^2,  u' = sqrt(2/pi)(1 + 3 0.044715 x^2).
constexpr float kSqrt2OverPi = 0.7978845608028654f;
constexpr float kGeluCubic = 0.044715f;
__device__ __forceinline__ void gelu_tanh_parts(float x, float& s, float& ar2) {
  // v = 2 u log2(e), so a = 2^{-|v|}
  const float v = x * fmaf(2.0f * kLog2e * kSqrt2OverPi * kGeluCubic, x * x,
                           2.0f * kLog2e * kSqrt2OverPi);
  const float a = __builtin_amdgcn_exp2f(-fabsf(v));
  const float r = __builtin_amdgcn_rcpf(1.0f + a);
  s = x < 0.0f ? a * r : r;
  ar2 = a * r * r;
}
__device__ __forceinline__ float gelu_tanh_f(float x) {
  float s, ar2;
  gelu_tanh_parts(x, s, ar2);
  return x * s;
}
__device__ __forceinline__ float gelu_tanh_grad(float x, float g) {
  float s, ar2;
  gelu_tanh_parts(x, s, ar2);
  const float du = kSqrt2OverPi * fmaf(3.0f * kGeluCubic, x * x, 1.0f);
  return g * fmaf(2.0f * x * du, ar2, s);
}

// ----------------------------------------------------------------------------------
// Host-side helpers shared by the C-ABI entry points.
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Attention operands: unit d-stride, (b, h, t) strides divisible by 4, 16-byte aligned base.
// Time strides (elements) of FP32 attention operands must lie in [0, kMaxAttnTimeStride).
constexpr int64_t kMaxAttnTimeStride = (int64_t)1 << 23;
bool attn_layout_ok(const float* p, const int64_t* s);
// Zero n floats with a fill kernel on `st`, not hipMemsetAsync: memset nodes recorded into a
// captured HIP graph have given wrong results on replays after the first.
int zero_floats(float* p, int64_t n, hipStream_t st);
// Validates (B, nh, T, hs) for the attention entry points; sets the error message on failure.
int check_attn_sizes(int64_t B, int64_t nh, int64_t T, int64_t hs);

}  // namespace cta
