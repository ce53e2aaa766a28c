/*
 * cuda_transformer_amd — C ABI of the MI355X (gfx950) FP32 transformer kernels.
 *
 * This is the drop-in boundary.  Each entry point replaces one launcher of the
 * reference's PyTorch extension (the .cu files of Transformer_launchers/) with plain
 * pointers, sizes and strides; no torch type appears here, so any FFI (ctypes, cgo, JNI,
 * N-API) can bind it.  The torch operator layer (cuda_transformer::* schemas) sits
 * on top of these functions.
 *
 * Conventions shared by every entry point
 *  - Tensors are FP32, device-resident (HIP device pointers).
 *  - Strides are in elements, outermost first.  Outputs are always dense
 *    row-major ("contiguous"), exactly as the reference launchers allocate them.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).  Every
 *    call is asynchronous on that stream; nothing synchronises the host.
 *  - Return value: CTA_OK (0) or one of the CTA_ERR_* codes; cta_last_error()
 *    then returns a message for the calling thread.  Messages for conditions the
 *    reference checks use the reference's wording.
 */
#ifndef CUDA_TRANSFORMER_AMD_H
#define CUDA_TRANSFORMER_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  CTA_OK = 0,
  CTA_ERR_INVALID_ARGUMENT = 1,     /* bad size / null pointer / mismatched shapes          */
  CTA_ERR_UNSUPPORTED_HEAD_DIM = 2, /* head size outside {32, 64, 128}                      */
  CTA_ERR_LAYOUT = 3,               /* stride or alignment the kernel cannot read directly   */
  CTA_ERR_LAUNCH = 4                /* the HIP runtime rejected a kernel launch              */
};

/* Message describing the last failure on the calling thread ("" if none). */
const char* cta_last_error(void);

/* Library version string. */
const char* cta_version(void);

/* ------------------------------------------------------------------------------
 * FlashAttention-2, FP32.  Shapes (B, nh, T, hs); hs in {32, 64, 128}.
 * softmax scale = 1/sqrt(hs) (the reference launcher passes sqrt(hs) and the
 * kernel inverts it: flash_attn_launcher.cu:27, flash_attention.cuh:45).
 * Q/K/V/O/dO strides: 4 entries (b, h, t, d).  The kernels need d-stride 1, other
 * strides divisible by 4, a t-stride in [0, 2^23) and 16-byte aligned base pointers
 * (CTA_ERR_LAYOUT otherwise; the torch layer passes a dense copy in that case).
 * L strides: 3 entries (b, h, t), any values.
 * ---------------------------------------------------------------------------- */

/* Forward: O (B,nh,T,hs) dense, L (B,nh,T) dense with L = rowmax + ln(rowsum).
 * Replaces cuda_transformer::flash_attention_fwd
 * (Transformer_launchers/flash_attn_launcher.cu:22-65). */
int cta_flash_attention_fwd(const float* q, const int64_t* q_strides,
                            const float* k, const int64_t* k_strides,
                            const float* v, const int64_t* v_strides,
                            int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                            float* o, float* l, void* stream);

/* Forward with O written through caller strides (4 entries (b, h, t, d), the same layout rules
 * as Q/K/V): e.g. straight into a (B, T, nh*hs) tensor, strides (T*nh*hs, hs, nh*hs, 1), which
 * the projection after attention reads without a transpose copy.  L dense as above.  Same
 * kernel and results as cta_flash_attention_fwd, which is this call with dense strides.  No
 * counterpart in the reference's launchers (their outputs are always dense); for callers with
 * packed (B, T, 3C) projections, such as the GPT harness. */
int cta_flash_attention_fwd_strided(const float* q, const int64_t* q_strides,
                                    const float* k, const int64_t* k_strides,
                                    const float* v, const int64_t* v_strides,
                                    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                    float* o, const int64_t* o_strides, float* l, void* stream);

/* Bytes of scratch with which cta_flash_attention_fwd_ex splits the forward's work:
 * (parts - 1)*B*nh*T*(hs+1) floats, parts = 2 or 3, when the grid would hold fewer than two
 * waves per SIMD of the MI355X (e.g. the B4 H4 N4096 D64 share of one GPU of eight); 0 when
 * the forward does not split. */
int64_t cta_flash_attention_fwd_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs,
                                          int causal);

/* cta_flash_attention_fwd_strided with a workspace.  Given cta_flash_attention_fwd_workspace()
 * bytes (when that is non-zero), each work item's K/V range is run by two or three workgroups,
 * which write the normalised partial O and L of their shares (part 0 into O and L, the others
 * into the workspace); a merge pass then combines them in a fixed order, L = ln(sum_k e^{Lk}),
 * O = sum_k e^{Lk-L} Ok.  Deterministic; equal to the unsplit forward to rounding.
 * Without the workspace (NULL or too small) it is cta_flash_attention_fwd_strided.  No
 * counterpart in the reference's launchers: their grid has no small-grid case to cover. */
int cta_flash_attention_fwd_ex(const float* q, const int64_t* q_strides,
                               const float* k, const int64_t* k_strides,
                               const float* v, const int64_t* v_strides,
                               int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                               float* o, const int64_t* o_strides, float* l,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* Forward with BF16 Q, K, V (stored as uint16_t bit patterns) and FP32 accumulation: O dense
 * (B,nh,T,hs) in BF16, L dense (B,nh,T) in FP32, L = rowmax + ln(rowsum) as above.  hs in
 * {32, 64, 128}.  Q/K/V strides: unit d-stride, other strides divisible by 8, a t-stride in
 * [0, 2^24), 16-byte aligned base pointers (CTA_ERR_LAYOUT otherwise).  The probabilities are rounded to BF16 as the
 * P.V operand.  No counterpart in the reference's launchers: its roadmap lists reduced
 * precision (README.md:277); the semantics are those of flash_attention_fwd
 * (flash_attn_launcher.cu:22-65). */
int cta_flash_attention_fwd_bf16(const uint16_t* q, const int64_t* q_strides,
                                 const uint16_t* k, const int64_t* k_strides,
                                 const uint16_t* v, const int64_t* v_strides,
                                 int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                 uint16_t* o, float* l, void* stream);

/* The same with FP16 Q, K, V (O in FP16, L in FP32; P rounded to FP16). */
int cta_flash_attention_fwd_f16(const uint16_t* q, const int64_t* q_strides,
                                const uint16_t* k, const int64_t* k_strides,
                                const uint16_t* v, const int64_t* v_strides,
                                int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                uint16_t* o, float* l, void* stream);

/* Bytes of dS workspace that let cta_flash_attention_bwd keep every head's dS tiles
 * (the lower-triangular 32x32 tiles only when causal): B*nh*ceil(T/32)^2*4 KiB, or about
 * half of that when causal.  0 for empty or unsupported shapes. */
int64_t cta_flash_attention_bwd_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs,
                                          int causal);

/* Extra workspace bytes with which cta_flash_attention_bwd splits a small grid's dK/dV and
 * dQ-from-dS stages (fewer than two waves per SIMD of the MI355X, T >= 1024): 2*B*nh*T*hs
 * floats for the second half's partial dK and dV, placed after every head's dS tiles, and
 * reused for the second half's partial dQ; 0 when the stages do not split.  Given
 * cta_flash_attention_bwd_workspace() + this many bytes, each key tile's query range (dK/dV)
 * and each query tile's key range (dQ) is run by two workgroups whose partial sums are then
 * added in a fixed order (deterministic; equal to the unsplit stages to rounding).  No
 * reference counterpart. */
int64_t cta_flash_attention_bwd_split_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs,
                                                int causal);

/* Backward: delta, then dQ and dK/dV.  dq/dk/dv are dense (B,nh,T,hs); `delta` is
 * caller-provided scratch of B*nh*T floats (the reference allocates it inside the launcher).
 * `workspace` may be NULL: the three stages then run as the reference schedules them, the
 * dQ stage recomputing S and dP.  Given at least one head's share of
 * cta_flash_attention_bwd_workspace() bytes, the dK/dV stage stores dS and dQ is computed
 * from it (cta_flash_attention_bwd_dkdv_store_ds + cta_flash_attention_bwd_dq_from_ds),
 * chunked over heads to fit workspace_bytes: fewer FLOPs, same results to rounding.
 * Both schedules are deterministic.
 * Replaces cuda_transformer::flash_attention_bwd (flash_attn_launcher.cu:67-142). */
int cta_flash_attention_bwd(const float* q, const int64_t* q_strides,
                            const float* k, const int64_t* k_strides,
                            const float* v, const int64_t* v_strides,
                            const float* o, const int64_t* o_strides,
                            const float* d_o, const int64_t* do_strides,
                            const float* l, const int64_t* l_strides,
                            int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                            float* dq, float* dk, float* dv, float* delta,
                            float* workspace, int64_t workspace_bytes, void* stream);

/* Backward with dQ, dK and dV written through caller strides (4 entries each, the same layout
 * rules as Q/K/V): e.g. into the three column blocks of one (B, T, 3*nh*hs) gradient of a
 * packed qkv projection.  Same kernels, schedules and results as cta_flash_attention_bwd,
 * which is this call with dense output strides.  No counterpart in the reference's launchers;
 * for callers with packed projections, such as the GPT harness. */
int cta_flash_attention_bwd_strided(const float* q, const int64_t* q_strides,
                                    const float* k, const int64_t* k_strides,
                                    const float* v, const int64_t* v_strides,
                                    const float* o, const int64_t* o_strides,
                                    const float* d_o, const int64_t* do_strides,
                                    const float* l, const int64_t* l_strides,
                                    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                    float* dq, const int64_t* dq_strides, float* dk,
                                    const int64_t* dk_strides, float* dv,
                                    const int64_t* dv_strides, float* delta, float* workspace,
                                    int64_t workspace_bytes, void* stream);

/* Largest B*nh*T that cta_flash_attention_bwd_noalloc accepts: 8,388,608 query rows, one float of
 * delta each in a 32 MiB device array. */
#define CTA_BWD_NOALLOC_MAX_ROWS 8388608

/* Allocation-free backward: the same gradients as cta_flash_attention_bwd with workspace NULL
 * (bitwise: the same kernels, delta then dQ recomputing S and dP then dK/dV), with no delta or
 * workspace argument.  delta lives in a file-scope device array of the library
 * (CTA_BWD_NOALLOC_MAX_ROWS floats, held on each GPU the library runs on until the process
 * ends); the call allocates no memory.  B*nh*T above CTA_BWD_NOALLOC_MAX_ROWS is rejected with
 * CTA_ERR_INVALID_ARGUMENT.  Calls that overlap on one GPU (different streams or host threads)
 * share that array and race.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). */
int cta_flash_attention_bwd_noalloc(const float* q, const int64_t* q_strides,
                                    const float* k, const int64_t* k_strides,
                                    const float* v, const int64_t* v_strides,
                                    const float* o, const int64_t* o_strides,
                                    const float* d_o, const int64_t* do_strides,
                                    const float* l, const int64_t* l_strides,
                                    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                    float* dq, float* dk, float* dv, void* stream);

/* Bytes of BF16 dS workspace for cta_flash_attention_bwd_bf16: B*nh*ceil(T/32)^2*2 KiB, or
 * about half of that when causal.  0 for empty or unsupported shapes (hs not in {32, 64, 128}). */
int64_t cta_flash_attention_bwd_bf16_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs,
                                               int causal);

/* Backward with BF16 Q, K, V, O, dO (uint16_t bit patterns) and FP32 L: delta (FP32, caller
 * scratch of B*nh*T floats), then dK/dV storing BF16 dS tiles and dQ from them, chunked over
 * heads to fit workspace_bytes.  With no workspace, or less than one head's share of
 * cta_flash_attention_bwd_bf16_workspace(), it runs the reference's schedule instead: a dQ
 * stage that recomputes S and dP (and forms delta, the same bits as the delta pass), then dK/dV
 * without the store (no O(T^2) memory; dK and dV bitwise equal to the stored schedule's, dQ
 * equal to rounding).  dq/dk/dv dense
 * (B,nh,T,hs) BF16.  hs in {32, 64, 128}; strides as for cta_flash_attention_fwd_bf16.  P and dS
 * are rounded to BF16 as MFMA operands; accumulation is FP32; deterministic.  No counterpart
 * in the reference's launchers (reduced precision is on its roadmap, README.md:277); the
 * semantics are those of flash_attention_bwd (flash_attn_launcher.cu:67-142). */
int cta_flash_attention_bwd_bf16(const uint16_t* q, const int64_t* q_strides,
                                 const uint16_t* k, const int64_t* k_strides,
                                 const uint16_t* v, const int64_t* v_strides,
                                 const uint16_t* o, const int64_t* o_strides,
                                 const uint16_t* d_o, const int64_t* do_strides,
                                 const float* l, const int64_t* l_strides,
                                 int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                 uint16_t* dq, uint16_t* dk, uint16_t* dv, float* delta,
                                 void* workspace, int64_t workspace_bytes, void* stream);

/* The same with FP16 Q, K, V, O, dO (FP32 L): FP16 gradients, dS stored and rounded in FP16. */
int64_t cta_flash_attention_bwd_f16_workspace(int64_t B, int64_t nh, int64_t T, int64_t hs,
                                              int causal);
int cta_flash_attention_bwd_f16(const uint16_t* q, const int64_t* q_strides,
                                const uint16_t* k, const int64_t* k_strides,
                                const uint16_t* v, const int64_t* v_strides,
                                const uint16_t* o, const int64_t* o_strides,
                                const uint16_t* d_o, const int64_t* do_strides,
                                const float* l, const int64_t* l_strides,
                                int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                uint16_t* dq, uint16_t* dk, uint16_t* dv, float* delta,
                                void* workspace, int64_t workspace_bytes, void* stream);

/* Stage 1 of the backward: delta[b,h,t] = sum_d O*dO, dense (B,nh,T).
 * Replaces the flash_attention_bwd_delta launch (flash_attn_launcher.cu:107-108). */
int cta_flash_attention_bwd_delta(const float* o, const int64_t* o_strides,
                                  const float* d_o, const int64_t* do_strides,
                                  int64_t B, int64_t nh, int64_t T, int64_t hs,
                                  float* delta, void* stream);

/* Stage 2: dQ.  Replaces the flash_attention_bwd_dq launch (flash_attn_launcher.cu:111,118,125). */
int cta_flash_attention_bwd_dq(const float* q, const int64_t* q_strides,
                               const float* k, const int64_t* k_strides,
                               const float* v, const int64_t* v_strides,
                               const float* d_o, const int64_t* do_strides,
                               const float* l, const int64_t* l_strides,
                               const float* delta,
                               int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                               float* dq, void* stream);

/* Stages 1 and 2 in one launch: dQ as cta_flash_attention_bwd_dq, forming delta itself from O
 * and dO (the same bits as cta_flash_attention_bwd_delta) and writing it to `delta` (dense
 * (B,nh,T)) for the dK/dV stage.  Replaces the flash_attention_bwd_delta and
 * flash_attention_bwd_dq launches (flash_attn_launcher.cu:107-108,111,118,125) of the
 * reference's schedule; cta_flash_attention_bwd runs it when it has no dS workspace. */
int cta_flash_attention_bwd_dq_delta(const float* q, const int64_t* q_strides,
                                     const float* k, const int64_t* k_strides,
                                     const float* v, const int64_t* v_strides,
                                     const float* o, const int64_t* o_strides,
                                     const float* d_o, const int64_t* do_strides,
                                     const float* l, const int64_t* l_strides,
                                     int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                     float* delta, float* dq, void* stream);

/* Stage 3: dK and dV.  Replaces the flash_attention_bwd_dk_dv launch
 * (flash_attn_launcher.cu:114,121,131). */
int cta_flash_attention_bwd_dkdv(const float* q, const int64_t* q_strides,
                                 const float* k, const int64_t* k_strides,
                                 const float* v, const int64_t* v_strides,
                                 const float* d_o, const int64_t* do_strides,
                                 const float* l, const int64_t* l_strides,
                                 const float* delta,
                                 int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                 float* dk, float* dv, void* stream);

/* Stage 3 of the stored-dS schedule: dK and dV as cta_flash_attention_bwd_dkdv, and every
 * dS tile written to ds_workspace (cta_flash_attention_bwd_workspace(B, nh, T, hs, causal)
 * bytes, 16-byte aligned).  Same launch slot as the reference's flash_attention_bwd_dk_dv
 * (flash_attn_launcher.cu:114,121,131), run before the dQ stage. */
int cta_flash_attention_bwd_dkdv_store_ds(const float* q, const int64_t* q_strides,
                                          const float* k, const int64_t* k_strides,
                                          const float* v, const int64_t* v_strides,
                                          const float* d_o, const int64_t* do_strides,
                                          const float* l, const int64_t* l_strides,
                                          const float* delta,
                                          int64_t B, int64_t nh, int64_t T, int64_t hs,
                                          int causal, float* dk, float* dv,
                                          float* ds_workspace, void* stream);

/* dQ = s * dS K from the tiles cta_flash_attention_bwd_dkdv_store_ds wrote.  Replaces the
 * flash_attention_bwd_dq launch (flash_attn_launcher.cu:111,118,125) in the stored-dS
 * schedule. */
int cta_flash_attention_bwd_dq_from_ds(const float* k, const int64_t* k_strides,
                                       const float* ds_workspace,
                                       int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                       float* dq, void* stream);

/* Backward with delta folded into the dK/dV stage: no delta launch and no delta scratch.  Each
 * dK/dV workgroup computes delta_i = O_i . dO_i for every query stage it visits from an O tile
 * streamed beside dO, stores dS, and dQ is computed from the stored tiles as in
 * cta_flash_attention_bwd (chunked over heads to fit workspace_bytes, which must hold at least
 * one head's share of cta_flash_attention_bwd_workspace(), else CTA_ERR_INVALID_ARGUMENT).
 * Same results to rounding (delta is summed in another order).  Folds the reference's
 * flash_attention_bwd_delta launch (flash_attn_launcher.cu:107-108, flash_attention.cuh:175-213)
 * into its flash_attention_bwd_dk_dv launch (flash_attn_launcher.cu:114,121,131); measured
 * slower than the separate delta launch, so cta_flash_attention_bwd does not use it. */
int cta_flash_attention_bwd_fold_delta(const float* q, const int64_t* q_strides,
                                       const float* k, const int64_t* k_strides,
                                       const float* v, const int64_t* v_strides,
                                       const float* o, const int64_t* o_strides,
                                       const float* d_o, const int64_t* do_strides,
                                       const float* l, const int64_t* l_strides,
                                       int64_t B, int64_t nh, int64_t T, int64_t hs, int causal,
                                       float* dq, float* dk, float* dv, float* workspace,
                                       int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------
 * Linear layer.
 * ---------------------------------------------------------------------------- */

/* Bytes of optional scratch for cta_cuda_fma (0 when the shape fills the GPU without a
 * K split). */
int64_t cta_cuda_fma_workspace(int64_t batch, int64_t m, int64_t k, int64_t n);

/* out[b] = x[b] . W[b or 0] + bias, out dense (batch, m, n).
 * x strides: 3 entries (batch, m, k).  W strides: 3 entries (batch, k, n); w_batch is 1
 * (broadcast, batch stride ignored) or `batch`.  Any strides: transposed views are read
 * in place.  `workspace` may be NULL; given cta_cuda_fma_workspace() bytes, shapes with few
 * output tiles and a long K are split along K with a deterministic reduction.  Outputs
 * are stored through 32-bit buffer offsets within a wave's block of rows; rows of 2^22 floats
 * and longer, which those offsets cannot span, are stored through 64-bit addresses instead.
 * Replaces cuda_transformer::cuda_fma (Transformer_launchers/linear_layer.cu:28-70). */
int cta_cuda_fma(const float* x, const int64_t* x_strides,
                 const float* w, const int64_t* w_strides,
                 const float* bias, int64_t bias_stride,
                 int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                 float* out, float* workspace, void* stream);

/* pre = x . W + bias and out = GELU(pre) (exact erf GELU) from one GEMM: the epilogue writes
 * both, so the activation costs no second pass over pre.  Arguments as cta_cuda_fma; pre and
 * out dense (batch, m, n), distinct; workspace sized by cta_cuda_fma_workspace().  Bitwise
 * equal to cta_cuda_fma followed by cta_gelu_fwd.  No single reference counterpart: it fuses
 * cuda_transformer::cuda_fma (linear_layer.cu:28-70) with gelu_activation
 * (gelu_activation.cu:22-47) as the GPT MLP composes them (gpt/gpt.py:133-136). */
int cta_cuda_fma_gelu(const float* x, const int64_t* x_strides,
                      const float* w, const int64_t* w_strides,
                      const float* bias, int64_t bias_stride,
                      int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                      float* pre, float* out, float* workspace, void* stream);

/* dx = (dy . W) * GELU'(pre), dx dense (batch, m, n); pre dense (batch, m, n), may alias dx.
 * dy and W as x and W of cta_cuda_fma (the GPT MLP passes fc2's W^T view).  Bitwise equal to
 * cta_cuda_fma with a zero bias followed by cta_gelu_bwd.  No single reference counterpart:
 * it fuses the dx product of CudaLinearLayer.backward (cuda_autograd_fns/
 * cuda_linear_layer.py:19-23) with gelu_activation_bwd (gelu_activation.cu:49-77). */
int cta_cuda_fma_gelu_grad(const float* dy, const int64_t* dy_strides,
                           const float* w, const int64_t* w_strides, const float* pre,
                           int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                           float* dx, float* workspace, void* stream);

/* As cta_cuda_fma_gelu with the tanh-approximated GELU: bitwise equal to cta_cuda_fma followed
 * by cta_gelu_tanh_fwd.  No reference counterpart (the reference's GELU is erf-exact,
 * GeLU.cuh:7-16); for MLPs that use the GPT-2 form. */
int cta_cuda_fma_gelu_tanh(const float* x, const int64_t* x_strides,
                           const float* w, const int64_t* w_strides,
                           const float* bias, int64_t bias_stride,
                           int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                           float* pre, float* out, float* workspace, void* stream);

/* As cta_cuda_fma_gelu_grad with the tanh-approximated GELU: bitwise equal to cta_cuda_fma with
 * a zero bias followed by cta_gelu_tanh_bwd.  No reference counterpart. */
int cta_cuda_fma_gelu_tanh_grad(const float* dy, const int64_t* dy_strides,
                                const float* w, const int64_t* w_strides, const float* pre,
                                int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                                float* dx, float* workspace, void* stream);

/* deriv = GELU'(x . W + bias) and out = GELU(x . W + bias) from one GEMM, arguments and
 * workspace as cta_cuda_fma_gelu (deriv in place of pre).  Saving the derivative instead of the
 * pre-activation moves the GELU' evaluation out of the backward product: cta_cuda_fma_mul with
 * this deriv is bitwise equal to cta_cuda_fma_gelu_grad with pre.  No single reference
 * counterpart (the same composition as cta_cuda_fma_gelu). */
int cta_cuda_fma_gelu_deriv(const float* x, const int64_t* x_strides,
                            const float* w, const int64_t* w_strides,
                            const float* bias, int64_t bias_stride,
                            int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                            float* deriv, float* out, float* workspace, void* stream);

/* As cta_cuda_fma_gelu_deriv with the tanh-approximated GELU (pairs with
 * cta_cuda_fma_gelu_tanh_grad).  No reference counterpart. */
int cta_cuda_fma_gelu_tanh_deriv(const float* x, const int64_t* x_strides,
                                 const float* w, const int64_t* w_strides,
                                 const float* bias, int64_t bias_stride,
                                 int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                                 float* deriv, float* out, float* workspace, void* stream);

/* dx = (dy . W) * d elementwise, d dense (batch, m, n), may alias dx; other arguments as
 * cta_cuda_fma_gelu_grad.  With d from cta_cuda_fma_gelu_deriv it is that op's GELU backward.
 * No single reference counterpart (the composition of cta_cuda_fma_gelu_grad). */
int cta_cuda_fma_mul(const float* dy, const int64_t* dy_strides,
                     const float* w, const int64_t* w_strides, const float* d,
                     int64_t batch, int64_t m, int64_t k, int64_t n, int64_t w_batch,
                     float* dx, float* workspace, void* stream);

/* dst[0..n) = src[0..n): a plain dwordx4 device copy (16-byte aligned buffers, n % 4 == 0), a
 * stream of one read and one write per element.  No counterpart in the reference: it is the
 * streaming ceiling that bench.py measures beside the bandwidth-bound kernels. */
int cta_device_copy(const float* src, float* dst, int64_t n, void* stream);

/* Bytes of scratch cta_db_calculation needs for a (batch, m, n) gradient. */
int64_t cta_db_calculation_workspace(int64_t batch, int64_t m, int64_t n);

/* db[n] = sum over (batch, m) of dy; dy strides: 3 entries.  Deterministic (no atomics).
 * Replaces cuda_transformer::db_calculation (linear_layer.cu:74-97). */
int cta_db_calculation(const float* dy, const int64_t* dy_strides,
                       int64_t batch, int64_t m, int64_t n,
                       float* db, float* workspace, void* stream);

/* Bytes of scratch cta_linear_weight_bias_grad needs. */
int64_t cta_linear_weight_bias_grad_workspace(int64_t rows, int64_t k, int64_t n);

/* dW = x^T dy (dense (k, n)) and db = column sums of dy (n), for x (rows, k) and dy (rows, n),
 * 2 strides each: the weight and bias gradients of CudaLinearLayer.backward with 2-D weights
 * (cuda_autograd_fns/cuda_linear_layer.py:21-27, the batch folded into the rows).  When dy is
 * n-contiguous with n % 4 == 0 and 16-byte aligned, db is summed inside the dW GEMM from the
 * dy slices it already loads (no second pass over dy); otherwise db comes from the
 * cta_db_calculation kernels.  dW is bitwise equal to cta_cuda_fma on the x^T view with a
 * zero bias; db differs from cta_db_calculation only in summation order.  Deterministic.
 * No single reference counterpart: it replaces the pair cuda_fma (dW) + db_calculation. */
int cta_linear_weight_bias_grad(const float* x, const int64_t* x_strides,
                                const float* dy, const int64_t* dy_strides,
                                int64_t rows, int64_t k, int64_t n,
                                float* dw, float* db, float* workspace, void* stream);

/* ------------------------------------------------------------------------------
 * Elementwise / row kernels (dense inputs, as the reference launchers require).
 * ---------------------------------------------------------------------------- */

/* y = x * Phi(x) (exact erf GELU).  Replaces cuda_transformer::gelu_activation
 * (Transformer_launchers/gelu_activation.cu:22-47). */
int cta_gelu_fwd(const float* x, float* y, int64_t numel, void* stream);

/* dx = dy * (Phi(x) + x * phi(x)).  Replaces cuda_transformer::gelu_activation_bwd
 * (gelu_activation.cu:49-77). */
int cta_gelu_bwd(const float* x, const float* dy, float* dx, int64_t numel, void* stream);

/* y = x * (1 + tanh(u)) / 2, u = sqrt(2/pi) * (x + 0.044715 x^3): torch's
 * F.gelu(x, approximate="tanh").  No reference kernel: the reference's GELU is erf-exact
 * (GeLU.cuh:7-16); this is the tanh-approximated GELU of the non-attention benchmark workload,
 * for models that use the GPT-2 form.  Same buffer rules as cta_gelu_fwd. */
int cta_gelu_tanh_fwd(const float* x, float* y, int64_t numel, void* stream);

/* dx = dy * d/dx [x * (1 + tanh(u)) / 2], as torch's tanh-GELU backward.  No reference
 * kernel (see cta_gelu_tanh_fwd). */
int cta_gelu_tanh_bwd(const float* x, const float* dy, float* dx, int64_t numel, void* stream);

/* Row softmax over `rows` rows of length n.  Replaces cuda_transformer::cuda_softmax
 * (Transformer_launchers/softmax_layer.cu:22-47). */
int cta_softmax_fwd(const float* x, float* y, int64_t rows, int64_t n, void* stream);

/* dx = p * (dp - sum(p * dp)) per row.  Replaces cuda_transformer::cuda_softmax_bwd
 * (softmax_layer.cu:50-78). */
int cta_softmax_bwd(const float* probs, const float* dp, float* dx,
                    int64_t rows, int64_t n, void* stream);

/* LayerNorm over the last dimension (no reference kernel; semantics of gpt/gpt.py:47-59):
 * y = (x - mean) * rstd * gamma + beta, rstd = 1/sqrt(biased var + eps).
 * Also writes mean and rstd (rows floats each) for the backward. */
int cta_layernorm_fwd(const float* x, const float* gamma, const float* beta,
                      int64_t rows, int64_t n, float eps,
                      float* y, float* mean, float* rstd, void* stream);

/* Bytes of scratch cta_layernorm_bwd needs. */
int64_t cta_layernorm_bwd_workspace(int64_t rows, int64_t n);

/* dx, dgamma, dbeta of the LayerNorm above.  Deterministic (no atomics). */
int cta_layernorm_bwd(const float* x, const float* gamma, const float* mean,
                      const float* rstd, const float* dy, int64_t rows, int64_t n,
                      float* dx, float* dgamma, float* dbeta, float* workspace, void* stream);

/* A residual add fused with the LayerNorm that follows it: xsum = x + f, y = LayerNorm(xsum)
 * (mean, rstd of xsum), one pass.  Bitwise equal to an elementwise add followed by
 * cta_layernorm_fwd.  No reference counterpart: the pre-LN block's `x + attn(...)` /
 * `x + mlp(...)` followed by the next LayerNorm (gpt/gpt.py:147-150, 47-59). */
int cta_add_layernorm_fwd(const float* x, const float* f, const float* gamma, const float* beta,
                          int64_t rows, int64_t n, float eps, float* xsum, float* y,
                          float* mean, float* rstd, void* stream);

/* Backward of cta_add_layernorm_fwd: dx = LayerNorm backward of dy at xsum, plus dres (the
 * gradient reaching xsum by the residual path); the gradient of both x and f.  dgamma, dbeta
 * as cta_layernorm_bwd; workspace from cta_layernorm_bwd_workspace.  Bitwise equal to
 * cta_layernorm_bwd followed by an elementwise add of dres.  No reference counterpart. */
int cta_add_layernorm_bwd(const float* xsum, const float* gamma, const float* mean,
                          const float* rstd, const float* dy, const float* dres, int64_t rows,
                          int64_t n, float* dx, float* dgamma, float* dbeta, float* workspace,
                          void* stream);

/* ------------------------------------------------------------------------------
 * Materialised causal self-attention (API parity with the reference's naive path).
 * ---------------------------------------------------------------------------- */

/* qkv dense (B, T, 3C); returns out dense (B, T, C) and probs dense (B, nh, T, T).
 * Replaces cuda_transformer::causal_self_attention_fwd
 * (Transformer_launchers/causal_self_attn_layer.cu:24-67). */
int cta_causal_self_attention_fwd(const float* qkv, int64_t B, int64_t T, int64_t C,
                                  int64_t nh, int causal, float* out, float* probs,
                                  void* stream);

/* Bytes of scratch cta_causal_self_attention_bwd needs (one (BH, T, T) buffer). */
int64_t cta_causal_self_attention_bwd_workspace(int64_t BH, int64_t T);

/* Q, K, V, dO: (BH, T, hs) with 3 strides each; probs dense (BH, T, T).  Returns dense
 * dq, dk (unscaled: the caller divides by sqrt(hs)) and dv.
 * Replaces cuda_transformer::causal_self_attention_bwd (causal_self_attn_layer.cu:70-132). */
int cta_causal_self_attention_bwd(const float* q, const int64_t* q_strides,
                                  const float* k, const int64_t* k_strides,
                                  const float* v, const int64_t* v_strides,
                                  const float* probs,
                                  const float* d_o, const int64_t* do_strides,
                                  int64_t BH, int64_t T, int64_t hs,
                                  float* dq, float* dk, float* dv, float* workspace,
                                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CUDA_TRANSFORMER_AMD_H */
