// Error reporting and version query of the C ABI.
#include "cta_common.hpp"

#include <string>

namespace cta {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(CTA_ERR_LAUNCH, std::string("Kernel Failed: ") + what + ": " + hipGetErrorString(err));
  return CTA_OK;
}

}  // namespace cta

extern "C" const char* cta_last_error(void) { return cta::g_last_error.c_str(); }

extern "C" const char* cta_version(void) { return "cuda_transformer_amd 0.1.0 (gfx950)"; }
