// abi_common.cpp — status codes and the thread-local error message of the
// C ABI.  The reference turns CUDA errors into std::runtime_error through
// CUDA_CHECK (tensor.h:28-34); across this C boundary the same information
// travels as a negative status plus msst_last_error().
#include <hip/hip_runtime.h>

#include <string>

#include "msst_common.hpp"

namespace msst {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(MSST_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
    return MSST_OK;
}

}  // namespace msst

extern "C" int msst_abi_version(void) { return 1; }

extern "C" const char* msst_status_string(int status) {
    switch (status) {
    case MSST_OK: return "ok";
    case MSST_ERR_INVALID_ARG: return "invalid argument";
    case MSST_ERR_UNSUPPORTED: return "unsupported shape or dtype";
    case MSST_ERR_ALIGNMENT: return "misaligned pointer";
    case MSST_ERR_LAUNCH: return "kernel launch failed";
    case MSST_ERR_WORKSPACE: return "workspace too small";
    default: return "unknown status";
    }
}

extern "C" const char* msst_last_error(void) { return msst::g_last_error.c_str(); }
