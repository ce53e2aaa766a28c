// Allocation-free FP32 FlashAttention-2 backward.
//
// cta_flash_attention_bwd takes its delta scratch (and the optional dS workspace) from the
// caller.  Callers that cannot allocate device memory at all (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc) call cta_flash_attention_bwd_noalloc
// instead: delta lives in the file-scope device array `scratch` below, and the backward runs
// the reference's schedule (dQ recomputing S and dP and forming delta, then dK/dV), which needs
// no other scratch.  The kernels are those of cta_flash_attention_bwd with a NULL workspace, so the
// results are bitwise identical to that call.
//
// The array is part of this library's code object: every GPU the library runs on holds its own
// copy (32 MiB) until the process ends.  Host code never passes `scratch` itself to a kernel
// (on the host that name is a stand-in, not a device address); it passes the device address
// hipGetSymbolAddress returns, resolved once per device on the first call with that device
// current.  Every call on one GPU shares that GPU's copy: calls that overlap on one GPU (two
// streams, or two host threads) race on delta.  Nothing in it needs to start at zero: the dQ
// kernel writes every entry the dK/dV kernel reads, in stream order.
#include "cta_common.hpp"

#include <mutex>

namespace cta {
namespace {

// delta needs one float per query row: B * nh * T <= CTA_BWD_NOALLOC_MAX_ROWS.
constexpr int64_t kScratchFloats = CTA_BWD_NOALLOC_MAX_ROWS;
static_assert(kScratchFloats * sizeof(float) == (int64_t{32} << 20), "scratch is 32 MiB");

static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, resolved on the first call per device.
int scratch_on_current_device(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(CTA_ERR_LAUNCH, "flash_attention_bwd_noalloc: no usable current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return fail(CTA_ERR_LAUNCH, std::string("flash_attention_bwd_noalloc: hipGetSymbolAddress "
                                              "of the scratch array failed: ") +
                                      hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return CTA_OK;
}

}  // namespace
}  // namespace cta

using namespace cta;

extern "C" int cta_flash_attention_bwd_noalloc(
    const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
    const float* v, const int64_t* v_strides, const float* o, const int64_t* o_strides,
    const float* d_o, const int64_t* do_strides, const float* l, const int64_t* l_strides,
    int64_t B, int64_t nh, int64_t T, int64_t hs, int causal, float* dq, float* dk, float* dv,
    void* stream) {
  if (int rc = check_attn_sizes(B, nh, T, hs)) return rc;
  if (B * nh * T == 0) return CTA_OK;
  if (B * nh * T > kScratchFloats)
    return fail(CTA_ERR_INVALID_ARGUMENT,
                "flash_attention_bwd_noalloc: B*nh*T = " + std::to_string(B * nh * T) +
                    " exceeds the allocation-free scratch (" + std::to_string(kScratchFloats) +
                    " rows of delta); call cta_flash_attention_bwd with caller-provided scratch");
  float* delta = nullptr;
  if (int rc = scratch_on_current_device(&delta)) return rc;
  return cta_flash_attention_bwd(q, q_strides, k, k_strides, v, v_strides, o, o_strides, d_o,
                                 do_strides, l, l_strides, B, nh, T, hs, causal, dq, dk, dv, delta,
                                 nullptr, 0, stream);
}
