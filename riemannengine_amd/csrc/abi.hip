// Error state and version of the C ABI (riemann_hip.h).
#include "rhip_internal.hpp"


namespace rhip {
static thread_local std::string g_last_error;
void set_last_error(const std::string &msg) { g_last_error = msg; }

// One pinned buffer per thread for read-backs of a few bytes (a copy to
// pageable memory goes through the runtime's staging copy and waits on it).
// A thread's calls run one after another, so no lock is held across the
// synchronisation and builds on other threads or GPUs are not serialised.
// Grown on demand; the buffer of a thread that exits is not reclaimed (at
// least 4 KiB of pinned memory per thread that ever read back).
// Kernels may write it directly through its device address (small results
// of a build's last kernel: no copy launch before the synchronisation); it
// is coherent (fine-grained) host memory, so those writes reach the host by
// the kernel's end.
static thread_local void *t_readback = nullptr;
static thread_local void *t_readback_dev = nullptr;
static thread_local size_t t_readback_bytes = 0;

PinnedReadback pinned_readback(size_t bytes) {
  if (t_readback_bytes < bytes) {
    void *p = nullptr;
    const size_t want = std::max<size_t>(bytes, 4096);
    RHIP_HIP(hipHostMalloc(&p, want, hipHostMallocMapped | hipHostMallocCoherent));
    if (t_readback)
      (void)hipHostFree(t_readback); // no copy uses it: this thread is here
    t_readback = p;
    t_readback_bytes = want;
    void *d = nullptr;
    if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess) {
      (void)hipGetLastError(); // not sticky: later launch checks must not see it
      d = nullptr;
    }
    t_readback_dev = d;
  }
  return PinnedReadback{t_readback, t_readback_dev};
}
} // namespace rhip

extern "C" const char *rhip_last_error(void) { return rhip::g_last_error.c_str(); }
extern "C" int rhip_abi_version(void) { return RHIP_ABI_VERSION; }
