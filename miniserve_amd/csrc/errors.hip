// C-ABI error state shared by every entry point.
#include "common.h"

namespace msa {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(MSA_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return MSA_OK;
}

}  // namespace msa

extern "C" const char* msa_last_error(void) { return msa::g_last_error.c_str(); }

extern "C" int msa_abi_version(void) { return 15; }
