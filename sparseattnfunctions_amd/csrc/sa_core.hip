// ABI version and per-thread error reporting for libsa_hip.so.
#include "sa_common.h"

namespace sa {
std::string& last_error_slot() {
  static thread_local std::string slot;
  return slot;
}
}  // namespace sa

extern "C" int sa_abi_version(void) { return SA_ABI_VERSION; }

extern "C" const char* sa_last_error(void) { return sa::last_error_slot().c_str(); }
