// C-ABI glue: per-thread error text and the ABI version of include/uttt_amd.h.
#include "uttt_host.h"

namespace uttt {
char* last_error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}
}  // namespace uttt

extern "C" const char* uttt_last_error(void) { return uttt::last_error_buffer(); }
extern "C" int uttt_abi_version(void) { return UTTT_ABI_VERSION; }
