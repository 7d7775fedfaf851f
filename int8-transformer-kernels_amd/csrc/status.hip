// status.hip — status codes, ABI version and per-thread error text of libint8k.
#include <string>

#include "int8k_common.h"

namespace int8k {

static thread_local std::string g_last_error;

void set_last_error(const char* what, hipError_t err) {
    g_last_error = std::string(what) + ": " + hipGetErrorName(err) + " (" +
                   hipGetErrorString(err) + ")";
}

void set_last_error_text(const char* text) { g_last_error = text; }

void clear_last_error() { g_last_error.clear(); }

}  // namespace int8k

extern "C" const char* int8k_status_string(int status) {
    switch (status) {
        case INT8K_OK: return "ok";
        case INT8K_ERR_INVALID_ARGUMENT: return "invalid argument";
        case INT8K_ERR_UNSUPPORTED: return "unsupported configuration";
        case INT8K_ERR_WORKSPACE: return "workspace missing or too small";
        case INT8K_ERR_MISALIGNED: return "pointer misaligned";
        case INT8K_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

extern "C" int int8k_abi_version(void) { return INT8K_ABI_VERSION; }

extern "C" const char* int8k_last_error(void) { return int8k::g_last_error.c_str(); }
