// Error reporting across the C ABI: a thread-local message per calling thread.
#include <string>

#include "../../include/yuf_engine.h"

namespace yuf {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int status, const std::string &msg) {
    g_last_error = msg;
    return status;
}

}  // namespace yuf

extern "C" const char *yuf_last_error(void) { return yuf::g_last_error.c_str(); }

extern "C" const char *yuf_version(void) { return "yufhip 0.1.0 (gfx950)"; }
