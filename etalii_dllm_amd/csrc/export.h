// Tensor files and fingerprints (export.hip): SHA-256 and the model.dllm / .dllmckpt byte layout.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

namespace dllm_hip {

class Sha256 {
  public:
    // impl: 0 the fastest available, 1 portable, 2 the x86 SHA extensions when the CPU has them
    explicit Sha256(int impl = 0);
    void update(const void* data, size_t n);
    void final_hex(char out[65]);

  private:
    void compress(const uint8_t* p, size_t blocks);
    uint32_t h_[8];
    uint8_t buf_[64];
    size_t fill_ = 0;
    uint64_t total_ = 0;
    bool ni_ = false;
};

// One tensor of a data section: numel float32 values in device or host memory.
struct TensorSource {
    const float* data;
    int64_t numel;
    bool device;
};

enum TensorFileKind { kModelFile = 0, kCheckpointFile = 1 };

// SHA-256 of the data section of `tensors` (each padded with zeros to 64 bytes); written to `file` when non-null.
int stream_tensor_data(const TensorSource* tensors, size_t n, FILE* file, char hex[65], hipStream_t stream);
// prefix + header (padded with spaces to a 64-byte data start) + data section; the header's 64-zero fingerprint
// placeholder is replaced by the data section's SHA-256, also returned in hex.
int write_tensor_file(const char* path, int kind, const char* header, size_t header_len, const TensorSource* tensors,
                      size_t n, char hex[65], hipStream_t stream);
// SHA-256 of a file's data section; with `load`, the tensors' destinations receive their bytes as they pass.
int read_tensor_file_data(const char* path, int kind, const TensorSource* tensors, size_t n, char hex[65], int load,
                          hipStream_t stream);

}  // namespace dllm_hip
