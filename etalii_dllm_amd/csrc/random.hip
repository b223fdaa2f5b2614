// Seeded synthetic inputs with the reference's generator (cpp/include/dllm/random.hpp, bound as kernels.cpp:130-136
// `Random` and kernels.cpp:206-218 `fill_gaussian`): xoshiro256** seeded through SplitMix64, doubles from the top
// 53 bits, and the Irwin-Hall Gaussian (12 uniforms - 6). Host code: the sequence of one seed is serial by nature;
// callers fill different tensors from different threads.
#include <stdint.h>

#include "common.h"
#include "dllm_hip.h"

namespace {

struct Xoshiro {
    uint64_t s[4];

    static uint64_t split_mix(uint64_t& state) {
        uint64_t z = (state += 0x9E3779B97F4A7C15ULL);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        return z ^ (z >> 31);
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

    explicit Xoshiro(uint64_t seed) {
        uint64_t sm = seed;
        for (int i = 0; i < 4; ++i) s[i] = split_mix(sm);
    }
    uint64_t next() {
        const uint64_t result = rotl(s[1] * 5, 7) * 9;
        const uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return result;
    }
    double next_double() { return static_cast<double>(next() >> 11) * (1.0 / 9007199254740992.0); }
    float next_gaussian() {
        double sum = 0.0;
        for (int i = 0; i < 12; ++i) sum += next_double();
        return static_cast<float>(sum - 6.0);
    }
};

}  // namespace

extern "C" {

int dllm_hip_fill_gaussian(uint64_t seed, float* host_out, size_t n, float scale) {
    DLLM_REQUIRE(host_out != nullptr || n == 0, "null output");
    Xoshiro r(seed);
    if (scale == 1.0f) {
        for (size_t i = 0; i < n; ++i) host_out[i] = r.next_gaussian();
    } else {
        for (size_t i = 0; i < n; ++i) host_out[i] = r.next_gaussian() * scale;
    }
    return dllm_hip::kOk;
}

int dllm_hip_random_tokens(uint64_t seed, int64_t* host_out, size_t n, int64_t vocab) {
    DLLM_REQUIRE(vocab > 0, "vocabulary must be positive");
    Xoshiro r(seed);
    for (size_t i = 0; i < n; ++i) host_out[i] = static_cast<int64_t>(r.next() % static_cast<uint64_t>(vocab));
    return dllm_hip::kOk;
}

}  // extern "C"
