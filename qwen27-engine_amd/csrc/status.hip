// Status reporting of the C ABI: int codes plus a per-thread message (q27h_last_error).
#include "q27h_internal.h"

namespace q27h {

static thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(Q27H_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return Q27H_OK;
}

}  // namespace q27h

extern "C" const char* q27h_last_error(void) { return q27h::g_last_error.c_str(); }
extern "C" int q27h_abi_version(void) { return Q27H_ABI_VERSION; }
