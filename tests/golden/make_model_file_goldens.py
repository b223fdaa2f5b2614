"""Writes tests/golden/model_file_header.json: model files written by the reference's own write_model_file
(src/etalii_dllm/modelfile.py:68-132) for two tiny architectures, as input/output vectors for the header bytes that no
reference fixture pins. Run in the build container only (it imports the reference from /root/reference/src; nothing
in the GPU runs or the product reads it):

    python3 tests/golden/make_model_file_goldens.py

Each case records the architecture dict (TransformerConfig.to_dict), the metadata, the tensor shapes, and what the
file holds: the header bytes after the 16-byte prefix (canonical JSON padded with spaces, the fingerprint patched
in), the fingerprint, and the SHA-256 of the whole file. The tensor values follow `tensor_values` below, which the
test restates.
"""

from __future__ import annotations

import hashlib
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

sys.path.insert(0, "/root/reference/src")
from etalii_dllm import modelfile  # noqa: E402
from etalii_dllm.architecture import TransformerConfig  # noqa: E402


def tensor_values(name: str, shape) -> np.ndarray:
    """Deterministic small floats, distinct per tensor: ((7 i + len(name)) mod 13 - 6) / 8."""
    n = int(np.prod(shape)) if len(shape) else 1
    i = np.arange(n, dtype=np.int64)
    return (((7 * i + len(name)) % 13 - 6).astype(np.float32) / np.float32(8)).reshape(shape)


CASES = {
    "llama_tied": (
        TransformerConfig(family="llama", vocabulary_size=64, hidden_size=16, intermediate_size=32, layers=2, heads=4,
                          kv_heads=2, head_dim=4, context_length=2048, rms_norm_eps=1e-5, rope_theta=100000.0,
                          tie_word_embeddings=True, bos_token_id=1, eos_token_ids=(2,)),
        {"source": {"format": "hf", "repository": "tiny/llama"}, "licence": {"id": "apache-2.0", "name": "Apache-2.0"},
         "tokenizer": None, "chat_template": "{{ messages }} — ünïcödé",
         "fine_tuning": {"steps_completed": 6, "final_loss": 0.1 + 0.2, "learning_rate": 1e-2}},
    ),
    "moe_post_norms": (
        TransformerConfig(family="olmoe", vocabulary_size=48, hidden_size=8, intermediate_size=12, layers=2, heads=2,
                          kv_heads=1, head_dim=4, context_length=512, rms_norm_eps=1e-6, rope_theta=10000.0,
                          qk_norm=True, qk_norm_scope="all", norm_placement="post", experts=4, experts_per_token=2,
                          expert_intermediate_size=6, normalize_expert_weights=False, eos_token_ids=(0, 3)),
        {"source": {"format": "gguf", "file": "x.gguf"}, "licence": None, "tokenizer": {"kind": "bpe"},
         "chat_template": None, "lineage": [{"step": "import", "source": {"format": "gguf"}}]},
    ),
}


def main() -> None:
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        for name, (config, metadata) in CASES.items():
            shapes = config.tensor_shapes()
            tensors = {n: modelfile.TensorSource(s, (lambda n=n, s=s: tensor_values(n, s))) for n, s in shapes.items()}
            path = Path(tmp) / f"{name}.dllm"
            fingerprint = modelfile.write_model_file(path, config, tensors, metadata)
            raw = path.read_bytes()
            length = int.from_bytes(raw[8:16], "little")
            out[name] = {
                "architecture": config.to_dict(),
                "metadata": metadata,
                "shapes": {n: list(s) for n, s in shapes.items()},
                "header": raw[16:16 + length].decode("utf-8"),
                "fingerprint": fingerprint,
                "file_sha256": hashlib.sha256(raw).hexdigest(),
                "file_bytes": len(raw),
            }
    target = Path(__file__).with_name("model_file_header.json")
    target.write_text(json.dumps(out, indent=1, ensure_ascii=False, sort_keys=True) + "\n", encoding="utf-8")
    print("wrote", target)


if __name__ == "__main__":
    main()
