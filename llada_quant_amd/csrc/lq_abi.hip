// lq_abi.hip -- version and error plumbing of the C ABI.
#include "lq_common.h"

namespace lq {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int status, const std::string &msg) {
  g_last_error = msg;
  return status;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(LQ_ERR_RUNTIME, std::string(what) + " launch failed: " + hipGetErrorString(e));
  return LQ_OK;
}

}  // namespace lq

extern "C" int lq_abi_version(void) { return LQ_ABI_VERSION; }

extern "C" const char *lq_last_error(void) { return lq::g_last_error.c_str(); }
