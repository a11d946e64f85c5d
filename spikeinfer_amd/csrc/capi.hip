// ABI-wide entry points: error message and version.
#include "common.hpp"

namespace spk {
std::string &last_error_slot() {
  static thread_local std::string msg;
  return msg;
}
}  // namespace spk

extern "C" const char *spk_last_error(void) { return spk::last_error_slot().c_str(); }

extern "C" int spk_abi_version(void) { return 3; }
