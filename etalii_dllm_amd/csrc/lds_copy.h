// Direct global -> LDS copies (gfx950 global_load_lds_dwordx4): each lane's 16 bytes land at M0 + 16 * lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dllm_hip {

// 16 bytes from src (a per-lane address) to LDS at lds_row + 16 * lane. Inline assembly, so the compiler's wait-count
// pass does not stall the LDS reads of the current stage on the in-flight copies of the next one; callers wait for
// their own copies explicitly.
__device__ __forceinline__ void copy16_to_lds(const void* src, const void* lds_row) {
    typedef __attribute__((address_space(3))) const void* lds_address;
    const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_address)lds_row));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// 16 bytes from sbase + voff (a wave-uniform base in SGPRs, a per-lane 32-bit byte offset) to LDS at
// lds_row + 16 * lane. No vector instruction is needed per copy when the offsets are computed once.
__device__ __forceinline__ void copy16_to_lds_s(const void* sbase, uint32_t voff, const void* lds_row) {
    typedef __attribute__((address_space(3))) const void* lds_address;
    const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_address)lds_row));
    // the base is wave-uniform; readfirstlane states it where the compiler cannot prove it
    const uint64_t a = reinterpret_cast<uint64_t>(sbase);
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32)));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu)));
    const uint64_t u = (static_cast<uint64_t>(hi) << 32) | lo;
    // s_nop 4: a vector instruction that wrote the base SGPRs (readfirstlane) must be 5 wait states ahead of a memory
    // instruction reading them, and the compiler's hazard checks do not look inside this statement
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(u), "{m0}"(m0) : "memory");
}

// 4 bytes from src (a per-lane address, 4-byte aligned) to LDS at lds_row + 4 * lane.
__device__ __forceinline__ void copy4_to_lds(const void* src, const void* lds_row) {
    typedef __attribute__((address_space(3))) const void* lds_address;
    const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_address)lds_row));
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// A workgroup barrier for LDS staged from registers: this wave's LDS writes complete (lgkmcnt), then s_barrier.
// Unlike __syncthreads(), whose release fence also waits for every outstanding global load, it leaves the loads of
// a register prefetch in flight across the barrier.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace dllm_hip
