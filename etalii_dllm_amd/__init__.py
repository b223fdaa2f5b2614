"""MI355X (gfx950) backend for EtAlii.Dllm's fine-tuning hot path: the backward pass and AdamW step behind
`dllm finetune`, as hand-written HIP kernels behind the C ABI of include/dllm_hip.h.

Submodules: kernels (the reference's kernel-module interface over the GPU), trainer (device-resident steps),
build (hipcc build of libdllm_hip.so).
"""

__all__ = ["kernels", "trainer", "build"]
