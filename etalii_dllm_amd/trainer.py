"""Device-resident fine-tuning steps on the MI355X: the host-side mirror of the reference's training loop pieces
(FineTuner._language_model_gradients and AdamW.step, src/etalii_dllm/training/trainer.py:290-335 and
training/optimizer.py:82-109) over the dllm_hip_trainer C ABI.

Weights, gradients, moments and activations stay on the GPU between steps; only token ids go in and the loss and
gradient norm come out.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from etalii_dllm_amd.kernels import check, lib

_i64p = C.POINTER(C.c_int64)


class DecoderConfig(C.Structure):
    """dllm_hip_decoder_config: the TransformerConfig fields a decoder step reads (architecture.py)."""

    _fields_ = [(name, C.c_int64) for name in (
        "vocab", "hidden", "intermediate", "layers", "heads", "kv_heads", "head_dim", "attention_bias", "qk_norm",
        "sliding_window", "tie_embeddings", "experts", "experts_per_token", "normalize_expert_weights",
        "expert_intermediate", "rotary_dim")] + [
        ("rms_norm_eps", C.c_double), ("rope_theta", C.c_double), ("attention_scale", C.c_double),
        ("embedding_multiplier", C.c_double), ("residual_multiplier", C.c_double), ("logits_scaling", C.c_double),
        ("dense_layers", C.c_int64), ("norm_placement", C.c_int64), ("norm_unit_offset", C.c_int64),
        ("activation", C.c_int64), ("full_attention_layers", C.c_int64), ("local_rope_theta", C.c_double),
        ("attention_softcap", C.c_double), ("logits_softcap", C.c_double), ("shared_inter", C.c_int64),
        ("shared_gate", C.c_int64), ("dense_layer_flags", C.POINTER(C.c_uint8)),
        ("full_attention_layer_flags", C.POINTER(C.c_uint8))]


class AdamWArgs(C.Structure):
    _fields_ = [(name, C.c_double) for name in (
        "learning_rate", "beta1", "beta2", "eps", "weight_decay", "max_grad_norm", "router_aux_loss")] + [
        ("step", C.c_int64)]


lib.dllm_hip_trainer_create.argtypes = [C.POINTER(DecoderConfig), C.c_int64, C.c_int64, C.c_int64,
                                        C.POINTER(C.c_void_p)]
lib.dllm_hip_trainer_destroy.argtypes = [C.c_void_p]


class LoraConfig(C.Structure):
    """dllm_hip_lora_config: LoraConfig (lora.py:159-177) with the targets as a mask and the base quantisation."""

    _fields_ = [("rank", C.c_int64), ("alpha", C.c_double), ("targets", C.c_int64), ("rslora", C.c_int64),
                ("base_quantize", C.c_int64)]


LORA_TARGET_BITS = {"q": 1, "k": 2, "v": 4, "o": 8, "gate": 16, "up": 32, "down": 64}


def lora_config(rank: int, alpha: float, targets=tuple(LORA_TARGET_BITS), rslora: bool = False,
                base_quantize: str | None = None) -> LoraConfig:
    kinds = {None: 0, "q8_0": 1, "q4_0": 2}
    if base_quantize not in kinds:
        raise ValueError(f"unknown base quantisation {base_quantize!r}; supported: q8_0, q4_0")
    mask = 0
    for t in targets:
        mask |= LORA_TARGET_BITS[t]
    return LoraConfig(rank, alpha, mask, int(rslora), kinds[base_quantize])


lib.dllm_hip_trainer_create_lora.argtypes = [C.POINTER(DecoderConfig), C.POINTER(LoraConfig), C.c_int64, C.c_int64,
                                             C.c_int64, C.POINTER(C.c_void_p)]
lib.dllm_hip_trainer_tensor.argtypes = [C.c_void_p, C.c_char_p, C.c_int, C.POINTER(C.c_void_p),
                                        C.POINTER(C.c_int64)]
lib.dllm_hip_trainer_tensor_count.argtypes = [C.c_void_p, C.POINTER(C.c_int64)]
lib.dllm_hip_trainer_gradients.argtypes = [C.c_void_p, _i64p, _i64p, _i64p, C.c_int64, C.c_double, C.c_double,
                                           C.POINTER(C.c_double), C.c_void_p]
lib.dllm_hip_trainer_router_loss.argtypes = [C.c_void_p, C.POINTER(C.c_double)]
lib.dllm_hip_trainer_set_rope.argtypes = [C.c_void_p, C.POINTER(C.c_double), C.c_int64, C.c_double]
lib.dllm_hip_trainer_step.argtypes = [C.c_void_p, _i64p, _i64p, _i64p, C.c_int64, C.POINTER(AdamWArgs),
                                      C.POINTER(C.c_double), C.POINTER(C.c_double), C.c_void_p]
lib.dllm_hip_trainer_dpo_step.argtypes = [C.c_void_p, _i64p, _i64p, _i64p, _i64p, C.c_int64, C.POINTER(C.c_double),
                                          C.c_double, C.POINTER(AdamWArgs), C.POINTER(C.c_double),
                                          C.POINTER(C.c_double), C.c_void_p]
lib.dllm_hip_trainer_log_probabilities.argtypes = [C.c_void_p, _i64p, _i64p, _i64p, _i64p, C.c_int64,
                                                   C.POINTER(C.c_double), C.c_void_p]


@dataclass(frozen=True)
class Decoder:
    """A pre-norm decoder's shape (architecture.py's TransformerConfig for the Llama/Qwen2/Qwen3 families)."""

    vocab: int
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    tie_embeddings: bool
    attention_bias: bool = False
    qk_norm: int = 0
    sliding_window: int = 0
    experts: int = 0  # routed experts per layer (Mixtral, OLMoE); 0 is a dense MLP
    experts_per_token: int = 0
    normalize_expert_weights: bool = False
    expert_intermediate: int = 0  # 0: the intermediate size
    rotary_dim: int = 0  # 0: head_dim (partial rotary: only the first rotary_dim dimensions of each head rotate)
    rope_scaling: dict | None = None  # a Hugging Face rope_scaling dict (linear, llama3, longrope or yarn)
    # Granite's multipliers (architecture.py's TransformerConfig, importer.py:427-434): attention_multiplier replaces
    # the attention scale 1/sqrt(head_dim)
    embedding_multiplier: float = 1.0
    attention_multiplier: float | None = None
    residual_multiplier: float = 1.0
    logits_scaling: float = 1.0
    dense_layers: tuple[int, ...] = ()  # layers keeping a dense MLP in a model with experts (Qwen3-MoE)
    norm_placement: int = 0  # 0 pre, 1 post (OLMo 2), 2 both (architecture.py:315-320)
    # Gemma: norms as 1 + w, GELU-tanh MLPs, the window on the layers in window_layers only (None: every layer), a RoPE
    # base of their own for those, soft-capped attention scores and logits
    norm_unit_offset: bool = False
    activation: int = 0  # 0 SiLU, 1 GELU (tanh approximation)
    window_layers: tuple[int, ...] | None = None
    local_rope_theta: float | None = None
    attention_softcap: float | None = None
    logits_softcap: float | None = None
    shared_inter: int = 0  # a shared expert's SwiGLU size in every routed layer (Qwen2-MoE, Granite MoE shared)
    shared_gate: bool = False  # its output times the sigmoid of a [1, hidden] gate (Qwen2-MoE)

    def native(self) -> DecoderConfig:
        # architecture.py:237-254 rejects layer indices outside the model
        if any(not 0 <= layer < self.layers for layer in self.dense_layers):
            raise ValueError("dense_layers must be layer indices")
        if self.window_layers is not None and any(not 0 <= layer < self.layers for layer in self.window_layers):
            raise ValueError("sliding_window_layers must be layer indices")
        # per-layer choices travel as one byte per layer (any depth); the 64-bit masks stay zero
        dense = (C.c_uint8 * self.layers)(*[int(layer in self.dense_layers) for layer in range(self.layers)])
        full = (C.c_uint8 * self.layers)(*[int(self.window_layers is not None and layer not in self.window_layers)
                                           for layer in range(self.layers)])
        cfg = DecoderConfig(self.vocab, self.hidden, self.intermediate, self.layers, self.heads, self.kv_heads,
                             self.head_dim, int(self.attention_bias), self.qk_norm, self.sliding_window,
                             int(self.tie_embeddings), self.experts, self.experts_per_token,
                             int(self.normalize_expert_weights), self.expert_intermediate,
                             self.rotary_dim or self.head_dim, self.rms_norm_eps, self.rope_theta,
                             1.0 / float(np.sqrt(np.float64(self.head_dim))) if self.attention_multiplier is None
                             else self.attention_multiplier, self.embedding_multiplier, self.residual_multiplier,
                             self.logits_scaling, 0, self.norm_placement, int(self.norm_unit_offset),
                             self.activation, 0, self.local_rope_theta or 0.0, self.attention_softcap or 0.0,
                             self.logits_softcap or 0.0, self.shared_inter, int(self.shared_gate),
                             C.cast(dense, C.POINTER(C.c_uint8)), C.cast(full, C.POINTER(C.c_uint8)))
        cfg._flags = (dense, full)  # kept alive with the structure until the trainer has read them
        return cfg


def _windows(windows):
    flat = np.ascontiguousarray([t for w in windows for t in w], dtype=np.int64)
    lengths = np.ascontiguousarray([len(w) for w in windows], dtype=np.int64)
    offsets = np.ascontiguousarray(np.concatenate([[0], np.cumsum(lengths)[:-1]]), dtype=np.int64)
    return flat, offsets, lengths


class Trainer:
    """One model's training state on the GPU."""

    PARAM, GRAD, M, V = 0, 1, 2, 3

    def __init__(self, decoder: Decoder, max_tokens: int, max_windows: int, max_window_tokens: int,
                 lora: LoraConfig | None = None) -> None:
        """lora: train LoRA adapters (tensors "<weight>.lora_a" / ".lora_b") on the frozen base instead."""
        self.decoder = decoder
        self.max_windows = max_windows
        self._cfg = decoder.native()
        self._lora = lora
        handle = C.c_void_p()
        check(lib.dllm_hip_trainer_create_lora(C.byref(self._cfg), C.byref(lora) if lora is not None else None,
                                               max_tokens, max_windows, max_window_tokens, C.byref(handle)))
        self.handle = handle
        count = C.c_int64()
        if decoder.rope_scaling:
            from etalii_dllm_amd.kernels import rope_attention_factor, rope_inv_freq

            inv = rope_inv_freq(decoder.head_dim, decoder.rope_theta, rotary_dim=decoder.rotary_dim or None,
                                scaling=decoder.rope_scaling)
            check(lib.dllm_hip_trainer_set_rope(handle, inv.ctypes.data_as(C.POINTER(C.c_double)), inv.size,
                                                rope_attention_factor(decoder.rope_scaling)))
        check(lib.dllm_hip_trainer_tensor_count(handle, C.byref(count)))
        self.names = [lib.dllm_hip_trainer_tensor_name(handle, i).decode() for i in range(count.value)]

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib.dllm_hip_trainer_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        self.close()

    def _tensor(self, name: str, which: int):
        ptr, numel = C.c_void_p(), C.c_int64()
        check(lib.dllm_hip_trainer_tensor(self.handle, name.encode(), which, C.byref(ptr), C.byref(numel)))
        return ptr, numel.value

    def set(self, name: str, values: np.ndarray, which: int = 0) -> None:
        a = np.ascontiguousarray(values, dtype=np.float32)
        ptr, numel = self._tensor(name, which)
        if a.size != numel:
            raise ValueError(f"{name}: expected {numel} values, got {a.size}")
        check(lib.dllm_hip_upload(ptr, a.ctypes.data, a.nbytes))

    def get(self, name: str, shape, which: int = 0) -> np.ndarray:
        ptr, numel = self._tensor(name, which)
        out = np.empty(shape, np.float32)
        if out.size != numel:
            raise ValueError(f"{name}: has {numel} values")
        check(lib.dllm_hip_download(out.ctypes.data, ptr, out.nbytes))
        return out

    def load(self, tensors: dict[str, np.ndarray], which: int = 0) -> None:
        for name, values in tensors.items():
            self.set(name, values, which)

    def gradients(self, windows, scale: float = 1.0, router_scale: float = 0.0) -> float:
        """DecoderGradients over each window, summed in window order; returns the summed loss (the summed router
        loss is `router_loss()` afterwards)."""
        flat, offsets, lengths = _windows(windows)
        loss = C.c_double()
        check(lib.dllm_hip_trainer_gradients(self.handle, flat.ctypes.data_as(_i64p), offsets.ctypes.data_as(_i64p),
                                             lengths.ctypes.data_as(_i64p), len(windows), scale, router_scale,
                                             C.byref(loss), None))
        return loss.value

    def router_loss(self) -> float:
        """The router load-balancing loss summed over the windows of the last gradients or step call."""
        value = C.c_double()
        check(lib.dllm_hip_trainer_router_loss(self.handle, C.byref(value)))
        return value.value

    def step(self, windows, learning_rate: float, step: int, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
             max_grad_norm=1.0, router_aux_loss=0.0) -> tuple[float, float]:
        """One fine-tuning step (trainer.py:290-310) at the given learning rate: (mean loss, gradient norm)."""
        flat, offsets, lengths = _windows(windows)
        args = AdamWArgs(learning_rate, beta1, beta2, eps, weight_decay, max_grad_norm, router_aux_loss, step)
        loss, norm = C.c_double(), C.c_double()
        check(lib.dllm_hip_trainer_step(self.handle, flat.ctypes.data_as(_i64p), offsets.ctypes.data_as(_i64p),
                                        lengths.ctypes.data_as(_i64p), len(windows), C.byref(args), C.byref(loss),
                                        C.byref(norm), None))
        return loss.value, norm.value

    # ---- files (modelfile.py, trainer.py:477-630) ----

    def fingerprint(self, kind: int = 0) -> str:
        """The SHA-256 of the data section the trainer would write: kind 0 the model file of weights() (equal to
        modelfile.data_fingerprint of the exported weights), kind 1 the checkpoint; streamed from device memory."""
        from etalii_dllm_amd.files import lib as flib

        out = C.create_string_buffer(65)
        check(flib.dllm_hip_trainer_fingerprint(self.handle, kind, out, None))
        return out.value.decode()

    def base_names(self) -> list[str]:
        """The model's tensors (weights()) in natural order."""
        return [n for n in self.names if not (n.endswith(".lora_a") or n.endswith(".lora_b"))]

    def trained_names(self) -> list[str]:
        """What AdamW updates: the adapters in a LoRA run, every tensor otherwise (natural order)."""
        if self._lora is None:
            return list(self.names)
        return [n for n in self.names if n.endswith(".lora_a") or n.endswith(".lora_b")]

    def export(self, path, architecture: dict, metadata: dict, shapes: dict) -> str:
        """FineTuner.export's file (trainer.py:477-509): `metadata` is the complete metadata the reference passes to
        write_model_file (with its fine_tuning and lineage sections); returns the fingerprint."""
        from etalii_dllm_amd import files

        header = files.model_header(architecture, shapes, metadata, self.base_names())
        out = C.create_string_buffer(65)
        check(files.lib.dllm_hip_trainer_write_file(self.handle, files.MODEL, str(path).encode(), header, len(header),
                                                    out, None))
        return out.value.decode()

    def save_checkpoint(self, path, shapes: dict, **fields) -> str:
        """FineTuner.save_checkpoint (trainer.py:524-568): fields are the header's architecture, run, step, losses,
        base_fingerprint, data_fingerprint, metadata (and reference); returns the checkpoint fingerprint."""
        from etalii_dllm_amd import files

        header = files.checkpoint_header(shapes=shapes, order=self.trained_names(), **fields)
        out = C.create_string_buffer(65)
        check(files.lib.dllm_hip_trainer_write_file(self.handle, files.CHECKPOINT, str(path).encode(), header,
                                                    len(header), out, None))
        return out.value.decode()

    def load_checkpoint(self, path, data_fingerprint: str | None = None) -> dict:
        """FineTuner.load_checkpoint's checks and restore (trainer.py:570-630) for this trainer's tensors: the data
        must match the header's fingerprint (and the run's data fingerprint, when given), the tensor list must be
        this trainer's. Returns the header (step, losses, run, metadata ...) for the caller's loop state."""
        from etalii_dllm_amd import files

        header = files.read_header(path, files.CHECKPOINT)
        if data_fingerprint is not None and header.get("data_fingerprint") != data_fingerprint:
            raise files.CheckpointError(f"{path}: the checkpoint was trained on different data")
        order = self.trained_names()
        want = [f"param/{n}" for n in order] + [f"{k}/{n}" for n in order for k in ("adam_m", "adam_v")]
        if [e["name"] for e in header.get("tensors", [])] != want:
            raise files.CheckpointError(f"{path}: the checkpoint holds other tensors than this run trains")
        status = files.lib.dllm_hip_trainer_read_checkpoint(self.handle, str(path).encode(),
                                                            str(header.get("fingerprint", "")).encode(), None)
        if status == 1:
            raise files.CheckpointError(lib.dllm_hip_last_error().decode())
        check(status)
        return header

    # ---- direct preference optimization (trainer.py:364-384, preference.py) ----

    @staticmethod
    def _pair_windows(pairs):
        """Windows 2p, 2p + 1: prompt + chosen and prompt + rejected tokens (PreferencePair.sequence)."""
        windows, prompts = [], []
        for prompt, chosen, rejected in pairs:
            windows += [[*prompt, *chosen], [*prompt, *rejected]]
            prompts.append(len(prompt))
        return windows, np.ascontiguousarray(prompts, dtype=np.int64)

    def log_probabilities(self, pairs) -> list[tuple[float, float]]:
        """(chosen, rejected) log-probabilities of each pair under the current weights (FineTuner.log_probability,
        trainer.py:443-453): the reference values of a DPO run when taken before its first step."""
        chunk = max(self.max_windows // 2, 1)  # pairs per call within the trainer's window capacity
        if len(pairs) > chunk:
            return [lp for i in range(0, len(pairs), chunk) for lp in self.log_probabilities(pairs[i:i + chunk])]
        windows, prompts = self._pair_windows(pairs)
        flat, offsets, lengths = _windows(windows)
        per_window = np.ascontiguousarray(np.repeat(prompts, 2), dtype=np.int64)
        out = np.zeros(len(windows), np.float64)
        check(lib.dllm_hip_trainer_log_probabilities(self.handle, flat.ctypes.data_as(_i64p),
                                                      offsets.ctypes.data_as(_i64p), lengths.ctypes.data_as(_i64p),
                                                      per_window.ctypes.data_as(_i64p), len(windows),
                                                      out.ctypes.data_as(C.POINTER(C.c_double)), None))
        return [(float(out[2 * p]), float(out[2 * p + 1])) for p in range(len(pairs))]

    def dpo_step(self, pairs, reference, beta: float, learning_rate: float, step: int, beta1=0.9, beta2=0.999,
                 eps=1e-8, weight_decay=0.01, max_grad_norm=1.0) -> tuple[float, float]:
        """One DPO step over `pairs` ((prompt, chosen, rejected) token tuples, in batch order) with their reference
        log-probabilities: (mean loss, gradient norm)."""
        windows, prompts = self._pair_windows(pairs)
        flat, offsets, lengths = _windows(windows)
        ref = np.ascontiguousarray(reference, dtype=np.float64).reshape(-1)
        args = AdamWArgs(learning_rate, beta1, beta2, eps, weight_decay, max_grad_norm, 0.0, step)
        loss, norm = C.c_double(), C.c_double()
        check(lib.dllm_hip_trainer_dpo_step(self.handle, flat.ctypes.data_as(_i64p), offsets.ctypes.data_as(_i64p),
                                             lengths.ctypes.data_as(_i64p), prompts.ctypes.data_as(_i64p),
                                             len(pairs), ref.ctypes.data_as(C.POINTER(C.c_double)), beta,
                                             C.byref(args), C.byref(loss), C.byref(norm), None))
        return loss.value, norm.value
