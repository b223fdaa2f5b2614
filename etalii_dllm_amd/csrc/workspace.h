// Carving one caller-provided workspace into typed, 256-byte aligned sub-buffers; Layout computes the bytes needed
// for the same sequence of takes.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace dllm_hip {

constexpr size_t kAlign = 256;

struct Layout {
    size_t bytes = 0;
    template <typename T>
    void add(size_t n) {
        bytes = (bytes + kAlign - 1) / kAlign * kAlign + (n > 0 ? n : 1) * sizeof(T);
    }
};

struct Carve {
    char* base;
    size_t used = 0, size;
    bool overflow = false;  // a take went past the workspace: the caller must not launch
    Carve(void* p, size_t bytes) : base(static_cast<char*>(p)), size(bytes) {}
    template <typename T>
    T* take(size_t n) {
        used = (used + kAlign - 1) / kAlign * kAlign;
        T* p = reinterpret_cast<T*>(base + used);
        used += (n > 0 ? n : 1) * sizeof(T);
        if (used > size) overflow = true;
        return p;
    }
};

}  // namespace dllm_hip
