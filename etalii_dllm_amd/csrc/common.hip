// Status and error-message plumbing shared by every entry point.
#include "common.h"

#include <string>

namespace dllm_hip {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string& message) { g_error = message; }
const char* last_error() { return g_error.c_str(); }

int fail(int status, const std::string& message) {
    set_error(message);
    return status;
}

int check_hip(hipError_t err, const char* what) {
    if (err == hipSuccess) return kOk;
    set_error(std::string(what) + ": " + hipGetErrorString(err));
    return err == hipErrorOutOfMemory ? kOutOfMemory : kHipError;
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

}  // namespace dllm_hip
