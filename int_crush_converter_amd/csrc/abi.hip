// Error state and version of the C ABI.
#include "common.hpp"

#include <cstring>

namespace icq {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

}  // namespace icq

extern "C" int ic_abi_version(void) { return IC_ABI_VERSION; }

extern "C" const char* ic_last_error(void) { return icq::g_last_error.c_str(); }
