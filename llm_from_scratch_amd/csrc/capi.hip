// ABI version and the thread-local error string of the C ABI.
#include "common.h"

namespace lfs {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

}  // namespace lfs

extern "C" int lfs_abi_version(void) { return LFS_ABI_VERSION; }
extern "C" const char* lfs_last_error(void) { return lfs::g_err; }
