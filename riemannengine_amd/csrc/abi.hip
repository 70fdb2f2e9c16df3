// Error state and version of the C ABI (riemann_hip.h).
#include "rhip_internal.hpp"

#include <mutex>

namespace rhip {
static thread_local std::string g_last_error;
void set_last_error(const std::string &msg) { g_last_error = msg; }

// One pinned buffer per process for read-backs of a few bytes: a copy to
// pageable memory goes through the runtime's staging copy and waits on it.
// Guarded by the lock in the returned holder; grown on demand, never freed.
static std::mutex g_readback_mutex;
static void *g_readback = nullptr;
static size_t g_readback_bytes = 0;

PinnedReadback pinned_readback(size_t bytes) {
  PinnedReadback r{std::unique_lock<std::mutex>(g_readback_mutex), nullptr};
  if (g_readback_bytes < bytes) {
    void *p = nullptr;
    const size_t want = std::max<size_t>(bytes, 4096);
    RHIP_HIP(hipHostMalloc(&p, want, hipHostMallocDefault));
    if (g_readback)
      (void)hipHostFree(g_readback); // unused: every user holds the lock
    g_readback = p;
    g_readback_bytes = want;
  }
  r.ptr = g_readback;
  return r;
}
} // namespace rhip

extern "C" const char *rhip_last_error(void) { return rhip::g_last_error.c_str(); }
extern "C" int rhip_abi_version(void) { return RHIP_ABI_VERSION; }
