// Thread-local error message of the C ABI.
#include <string>

#include "../../include/mi355moe.h"

namespace mi355 {
namespace {
thread_local std::string g_last_error;
}
int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
}  // namespace mi355

extern "C" const char* mi355moe_last_error(void) {
  return mi355::g_last_error.c_str();
}

extern "C" int mi355moe_version(void) { return 1; }
