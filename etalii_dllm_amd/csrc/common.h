// Shared plumbing of the HIP library: status codes, the per-thread error message, launch checks and small helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace dllm_hip {

// A pointer restated as addressing global memory. A copy the compiler cannot follow (e.g. one passed through inline
// assembly to keep it in scalar registers) loses that, and its loads and stores become flat ones, which wait on both
// the vector-memory and the LDS counters.
template <typename T>
using global_pointer = __attribute__((address_space(1))) T*;

template <typename T>
__device__ __forceinline__ global_pointer<T> global_ptr(T* p) {
    return (global_pointer<T>)p;
}

enum Status : int {
    kOk = 0,
    kInvalidArgument = 1,  // the reference raises ValueError for these (cpp/kernels.cpp:97-101)
    kHipError = 2,
    kOutOfMemory = 3,
};

// The message of the last failure on the calling thread (dllm_hip_last_error).
void set_error(const std::string& message);
const char* last_error();

int fail(int status, const std::string& message);

// Returns kOk or records the HIP error of the last launch / call.
int check_hip(hipError_t err, const char* what);
int check_launch(const char* what);

inline size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }
inline size_t round_up(size_t a, size_t b) { return ceil_div(a, b) * b; }

// Wave size of CDNA: every kernel here is written for 64-wide wavefronts.
constexpr int kWave = 64;

}  // namespace dllm_hip

#define DLLM_TRY(expr)                      \
    do {                                    \
        const int dllm_status_ = (expr);    \
        if (dllm_status_ != 0) return dllm_status_; \
    } while (0)

#define DLLM_REQUIRE(cond, message)                                                \
    do {                                                                           \
        if (!(cond)) return ::dllm_hip::fail(::dllm_hip::kInvalidArgument, message); \
    } while (0)
