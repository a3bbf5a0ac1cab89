// common.cpp — error state and version of the cortexsdr_amd C-ABI.
#include "common.hpp"

namespace csdr {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

const char* last_error() { return g_last_error.c_str(); }

}  // namespace csdr

extern "C" {

CSDR_API const char* csdr_last_error(void) { return csdr::last_error(); }

CSDR_API const char* csdr_version(void) { return "cortexsdr_amd 0.1.0 (gfx950)"; }

}
