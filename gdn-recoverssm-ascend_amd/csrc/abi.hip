// ABI version and the thread-local error channel of the C entry points.
#include <atomic>
#include <cstdarg>
#include <cstdio>

#include "gdn_common.cuh"

namespace gdn {

static thread_local char g_last_error[512] = "";
static std::atomic<int64_t> g_state_retain{GDN_STATE_CACHE_RETAIN_DEFAULT};

int64_t state_cache_retain() { return g_state_retain.load(std::memory_order_relaxed); }

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace gdn

extern "C" int gdn_recoverssm_abi_version(void) { return GDN_RECOVERSSM_ABI_VERSION; }

extern "C" const char *gdn_recoverssm_last_error(void) { return gdn::g_last_error; }

extern "C" int64_t gdn_recoverssm_set_state_cache_retain(int64_t bytes) {
  if (bytes < 0) return -1;
  return gdn::g_state_retain.exchange(bytes, std::memory_order_relaxed);
}
