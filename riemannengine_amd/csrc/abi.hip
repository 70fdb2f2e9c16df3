// Error state and version of the C ABI (riemann_hip.h).
#include "rhip_internal.hpp"

namespace rhip {
static thread_local std::string g_last_error;
void set_last_error(const std::string &msg) { g_last_error = msg; }
} // namespace rhip

extern "C" const char *rhip_last_error(void) { return rhip::g_last_error.c_str(); }
extern "C" int rhip_abi_version(void) { return RHIP_ABI_VERSION; }
