// ABI version and the thread-local error channel of the C entry points.
#include <cstdarg>
#include <cstdio>

#include "gdn_common.cuh"

namespace gdn {

static thread_local char g_last_error[512] = "";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace gdn

extern "C" int gdn_recoverssm_abi_version(void) { return GDN_RECOVERSSM_ABI_VERSION; }

extern "C" const char *gdn_recoverssm_last_error(void) { return gdn::g_last_error; }
