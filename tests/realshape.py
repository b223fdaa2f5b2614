"""The benchmark configurations at their real layer shapes, for bitwise parity of the GPU step with the oracle's step
over the reference kernels (oracle/_ref): the configurations, a fast seeded input generator both sides share, and the
per-tensor SHA-256 digests a run is compared by.

The oracle's step at these shapes takes minutes of CPU time (the reference's head matmuls and its single-threaded
cross-entropy, attention backward and AdamW), so tests/golden/make_realshape_goldens.py runs it once and commits the
digests of every gradient, parameter and AdamW moment after each step (tests/golden/realshape_<name>.json); the GPU
test regenerates the same inputs, runs the same steps on the GPU and compares digests. Equal SHA-256 digests are equal
bits.

Shapes follow BASELINE's configurations (SmolLM2-135M, Qwen2.5-1.5B, Qwen3-0.6B with LoRA on a Q8_0 base, OLMoE-1B-7B),
plus Gemma-2-2B's layer (256-wide heads, soft-caps, sandwich norms, vocabulary 256000) Qwen1.5-MoE-A2.7B's (60
experts and a gated shared expert) and OLMo-2-1B's (post norms), with fewer layers where the full depth only repeats the same launches; the vocabulary, hidden size, heads,
intermediate sizes, window lengths and expert counts are the real ones, so every size-selected code path of the step
(matmul grid layouts, the windows-in-sequence tied-embedding dW, the transposes, the window sums, the attention tiles
at T = 2048, the cross-entropy at vocab 151936, the grouped expert matmuls) runs at the shape it runs at in the bench.
"""

from __future__ import annotations

import hashlib
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, replace

import numpy as np

import oracle_lib as O


@dataclass(frozen=True)
class RealShape:
    name: str
    decoder: O.Decoder
    windows: tuple[int, ...]  # tokens per window (inputs + 1)
    steps: int = 1
    lora: O.Lora | None = None
    base_quantize: str | None = None
    router_aux_loss: float = 0.0
    learning_rate: float = 1e-4
    seed: int = 0
    notes: str = ""


def _configs() -> dict[str, RealShape]:
    smollm = O.Decoder("llama", vocab=49152, hidden=576, inter=1536, layers=30, heads=9, kv_heads=3, head_dim=64,
                       eps=1e-5, rope_theta=1e5, tied=True)
    qwen25 = O.Decoder("qwen2", vocab=151936, hidden=1536, inter=8960, layers=2, heads=12, kv_heads=2, head_dim=128,
                       eps=1e-6, rope_theta=1e6, tied=True, attn_bias=True)
    qwen3 = O.Decoder("qwen3", vocab=151936, hidden=1024, inter=3072, layers=2, heads=16, kv_heads=8, head_dim=128,
                      eps=1e-6, rope_theta=1e6, tied=True, qk_norm=1)
    olmoe = O.Decoder("olmoe", vocab=50304, hidden=2048, inter=1024, layers=1, heads=16, kv_heads=16, head_dim=128,
                      eps=1e-5, rope_theta=1e4, tied=False, qk_norm=2, experts=64, topk=8, normalize=False,
                      expert_inter=1024)
    gemma2 = O.Decoder("gemma2", vocab=256000, hidden=2304, inter=9216, layers=2, heads=8, kv_heads=4, head_dim=256,
                       eps=1e-6, rope_theta=1e4, tied=True, norm_placement=2, unit_offset=True, activation=1,
                       window=300, window_layers=(0,), embedding_multiplier=float(np.sqrt(2304.0)),
                       attention_multiplier=256.0 ** -0.5, attention_softcap=50.0, logits_softcap=30.0)
    qwen2_moe = O.Decoder("qwen2_moe", vocab=151936, hidden=2048, inter=5632, layers=1, heads=16, kv_heads=16,
                          head_dim=128, eps=1e-6, rope_theta=1e6, tied=False, attn_bias=True, experts=60, topk=4,
                          normalize=False, expert_inter=1408, shared_inter=5632, shared_gate=True)
    olmo2 = O.Decoder("olmo2", vocab=100352, hidden=2048, inter=8192, layers=2, heads=16, kv_heads=16, head_dim=128,
                      eps=1e-6, rope_theta=5e5, tied=False, qk_norm=2, norm_placement=1)
    return {
        "olmo2": RealShape("olmo2", olmo2, (1025, 257), seed=8,
                           notes="OLMo-2-1B layer shapes, 2 of 16 layers, post norms and whole-projection QK-norm, "
                                 "windows of 1024 and 256"),
        "qwen2_moe": RealShape("qwen2_moe", qwen2_moe, (513, 257), router_aux_loss=0.001, seed=7,
                               notes="Qwen1.5-MoE-A2.7B layer shapes, 1 of 24 layers, 60 experts top 4 with the gated "
                                     "shared expert of 5632, windows of 512 and 256, router_aux_loss 0.001"),
        "gemma2": RealShape("gemma2", gemma2, (513, 257), seed=6,
                            notes="Gemma-2-2B layer shapes, 2 of 26 layers (one windowed, one global), vocabulary "
                                  "256000, 256-wide heads, soft-capped scores and logits, windows of 512 and 256"),
        "c1": RealShape("c1", smollm, (257, 257, 257, 257), steps=2, seed=1,
                        notes="SmolLM2-135M, full depth, 4 x 256 tokens, two steps"),
        "c3": RealShape("c3", qwen25, (1025,) * 8, seed=3,
                        notes="Qwen2.5-1.5B layer shapes, 2 of 28 layers, full vocabulary, the bench's 8 x 1024 "
                              "tokens"),
        "c4": RealShape("c4", qwen3, (2049, 2049, 2049, 701), steps=2, lora=O.Lora(rank=16, alpha=32.0),
                        base_quantize="q8_0", seed=4, learning_rate=1e-3,
                        notes="Qwen3-0.6B layer shapes, 2 of 28 layers, LoRA r16 on all 7 targets over a Q8_0 base, "
                              "windows of 2048, 2048, 2048 and 700 tokens, two steps (B non-zero)"),
        "c5": RealShape("c5", olmoe, (2049, 501), router_aux_loss=0.01, seed=5,
                        notes="OLMoE-1B-7B layer shapes, 1 of 16 layers, 64 experts top 8, windows of 2048 and 500 "
                              "tokens, router_aux_loss 0.01"),
        "c5_depth": RealShape("c5_depth", replace(olmoe, layers=16), (129, 65), router_aux_loss=0.01, seed=9,
                              notes="OLMoE-1B-7B at full depth: all 16 layers, the whole 6.92 B-parameter arena "
                                    "(more than 2^32 values per arena, 3219 tensors in the AdamW chunk table and "
                                    "the exact-norm plan), windows of 128 and 64 tokens, router_aux_loss 0.01"),
    }


CONFIGS = _configs()
WORKERS = min(16, os.cpu_count() or 1)

_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


def uniform(seed: int, n: int, std: float) -> np.ndarray:
    """n float32 values, uniform with standard deviation std: the SplitMix64 finaliser of (index + seed * golden
    ratio), its top 24 bits as u in [0, 1), then (u - 0.5) * f32(std * sqrt(12)). Fast and the same on every
    machine (integer arithmetic, then exact or single-rounded float32 operations)."""
    out = np.empty(n, np.float32)
    width = np.float32(std * np.sqrt(12.0))
    chunk = 1 << 24
    with np.errstate(over="ignore"):
        for start in range(0, n, chunk):
            z = np.arange(start, min(n, start + chunk), dtype=np.uint64) + np.uint64(seed) * _GOLDEN
            z = (z ^ (z >> np.uint64(30))) * _M1
            z = (z ^ (z >> np.uint64(27))) * _M2
            z ^= z >> np.uint64(31)
            u = (z >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
            out[start:start + u.size] = (u - np.float32(0.5)) * width
    return out


def weights(cfg: RealShape) -> dict[str, np.ndarray]:
    """Parameters in natural order: norms 1.0, everything else uniform with std 0.02 (routers 0.1, so the top-k
    choices spread), seeded per tensor."""
    shapes = cfg.decoder.tensor_shapes()
    names = O.tensor_order(shapes)

    def make(index: int) -> np.ndarray:
        name = names[index]
        shape = shapes[name]
        if name.endswith("norm.weight"):
            return np.ones(shape, np.float32)
        std = 0.1 if name.endswith("router.weight") else 0.02
        return uniform(cfg.seed * 100003 + index, int(np.prod(shape)), std).reshape(shape)

    # tensors are independent (each seeded by its index): generated on a thread pool (numpy releases the GIL)
    with ThreadPoolExecutor(max_workers=WORKERS) as pool:
        values = list(pool.map(make, range(len(names))))
    return dict(zip(names, values))


def adapters(cfg: RealShape) -> dict[str, np.ndarray]:
    """LoRA adapters in natural order, A and B both non-zero (std 0.02) so the merge and both adapter gradients
    carry signal from the first step."""
    shapes = O.adapter_shapes(cfg.decoder, cfg.lora)
    return {name: uniform(cfg.seed * 100003 + 50000 + index, int(np.prod(shape)), 0.02).reshape(shape)
            for index, (name, shape) in enumerate(shapes.items())}


def windows(cfg: RealShape) -> list[list[int]]:
    """Token windows: Random(seed).next_u64() % vocab (random.hpp's xoshiro256**), window after window."""
    rng = O.Random(cfg.seed)
    return [[rng.next_u64() % cfg.decoder.vocab for _ in range(n)] for n in cfg.windows]


def quantized_base(cfg: RealShape, base: dict[str, np.ndarray], quantize) -> dict[str, np.ndarray]:
    """QuantizedBase (lora.py:300-302): the q k v o gate up down matrices whose input size is a multiple of 32 as
    their Q8_0-dequantised values; quantize is a quantize_q8_0(x, q, scales, n) C function."""
    out = dict(base)
    for name, shape in cfg.decoder.tensor_shapes().items():
        if name.endswith((".q.weight", ".k.weight", ".v.weight", ".o.weight", ".gate.weight", ".up.weight",
                          ".down.weight")) and len(shape) == 2 and shape[1] % 32 == 0:
            q, s = O.quantize_q8_0(quantize, base[name])
            out[name] = O.dequantize_q8_0(q, s).reshape(shape)
    return out


def digest(values: np.ndarray) -> str:
    return hashlib.sha256(memoryview(np.ascontiguousarray(values, dtype=np.float32)).cast("B")).hexdigest()


def digest_of_concatenation(arrays) -> str:
    """digest(np.concatenate of the arrays' flattened values), without forming the concatenation."""
    h = hashlib.sha256()
    for a in arrays:
        h.update(memoryview(np.ascontiguousarray(a, dtype=np.float32)).cast("B"))
    return h.hexdigest()


def double_hex(x: float) -> str:
    return float(x).hex()
