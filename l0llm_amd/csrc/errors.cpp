// Status messages of libl0hip (host only): the thread-local text behind l0h_last_error. Kept apart
// from the HIP runtime so the host-side C++ (quantizer, RoPE tables, safetensors reader) also
// builds and runs on its own, e.g. under the address and undefined-behaviour sanitizers.
#include <string>

#include "../../include/l0hip.h"

namespace l0h {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

}  // namespace l0h

extern "C" const char* l0h_last_error(void) { return l0h::g_last_error.c_str(); }
