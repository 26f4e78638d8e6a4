// Library-wide C ABI pieces: version and per-thread error text.
#include "cda_common.h"

namespace cda {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string &msg) { g_last_error = msg; }

}  // namespace cda

extern "C" int cda_hip_version(void) { return 100; }

extern "C" const char *cda_hip_last_error(void) { return cda::g_last_error.c_str(); }
