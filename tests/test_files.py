"""Model and checkpoint files without a GPU: the library's SHA-256 against hashlib and the FIPS 180-4 examples, and the
byte layout of its writer against a restatement of the reference's write_model_file and save_checkpoint
(src/etalii_dllm/modelfile.py:68-136, training/trainer.py:524-568) on host tensors."""

from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

LIBRARY = Path(__file__).resolve().parents[1] / "etalii_dllm_amd" / "libdllm_hip.so"
pytestmark = pytest.mark.skipif(not LIBRARY.exists(), reason="libdllm_hip.so not built")


@pytest.fixture(scope="module")
def F():
    from etalii_dllm_amd import files

    return files


# FIPS 180-4 / NIST example messages
VECTORS = {
    b"": "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855",
    b"abc": "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad",
    b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq":
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
}


@pytest.mark.parametrize("impl", [0, 1, 2])
def test_sha256_known_answers_and_hashlib(F, impl):
    for message, digest in VECTORS.items():
        assert F.sha256(message, impl) == digest
    assert F.sha256(b"a" * 1_000_000, impl) == "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"
    rng = np.random.default_rng(1)
    for n in [1, 55, 56, 63, 64, 65, 119, 120, 127, 128, 129, 1000, 4097, (1 << 20) + 3]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert F.sha256(data, impl) == hashlib.sha256(data).hexdigest(), n


def reference_layout(kind: int, header: bytes, tensors) -> tuple[bytes, str]:
    """The file write_model_file / save_checkpoint produce for `header` (canonical JSON with the 64-zero placeholder)
    and the tensors in order: prefix, header padded with spaces to a 64-byte data start, each tensor's float32 bytes
    padded with zeros to 64, the data section's SHA-256 patched into the placeholder (modelfile.py:119-136,238-243;
    trainer.py:559-568)."""
    prefix = struct.Struct("<4sIQ") if kind == 0 else struct.Struct("<8sIQ")
    magic = b"DLLM" if kind == 0 else b"DLLMCKPT"
    padded = header + b" " * (-(prefix.size + len(header)) % 64)
    data = b""
    for t in tensors:
        raw = np.ascontiguousarray(t, dtype="<f4").tobytes()
        data += raw + b"\0" * (-len(raw) % 64)
    fingerprint = hashlib.sha256(data).hexdigest()
    marker = b'"fingerprint":"' + b"0" * 64 + b'"'
    at = padded.index(marker) + len(b'"fingerprint":"')
    padded = padded[:at] + fingerprint.encode() + padded[at + 64:]
    return prefix.pack(magic, 1, len(padded)) + padded + data, fingerprint


def tiny_tensors():
    rng = np.random.default_rng(3)
    shapes = {"layers.10.w": (3, 5), "layers.2.w": (7,), "embedding": (16, 4), "norm": (1,), "empty": (0,)}
    return shapes, {n: rng.standard_normal(s).astype(np.float32) for n, s in shapes.items()}


@pytest.mark.parametrize("kind", [0, 1])
def test_writer_matches_the_reference_layout(F, tmp_path, kind):
    shapes, values = tiny_tensors()
    order = ["embedding", "empty", "layers.2.w", "layers.10.w", "norm"]
    if kind == 0:
        metadata = {"source": {"format": "hf", "repository": "x/y"}, "licence": {"id": "apache-2.0"},
                    "tokenizer": None, "chat_template": "{{ m }}", "fine_tuning": {"steps_completed": 6}}
        header = F.model_header({"family": "llama", "hidden": 4}, shapes, metadata, order)
        tensors = [values[n] for n in order]
    else:
        header = F.checkpoint_header(architecture={"family": "llama"}, run={"steps": 6, "objective": "lm"}, step=3,
                                     losses=[1.5, 0.1 + 0.2], base_fingerprint="b" * 64, data_fingerprint="d" * 64,
                                     metadata={"lineage": []}, shapes=shapes, order=order,
                                     reference=[(0.5, 1.0 / 3.0)])
        tensors = [values[n] for n in order] + [values[n] * k for n in order for k in (2.0, 3.0)]
    want, fingerprint = reference_layout(kind, header, tensors)
    path = tmp_path / ("model.dllm" if kind == 0 else "run.dllmckpt")
    assert F.write_tensor_file(path, kind, header, tensors) == fingerprint
    assert path.read_bytes() == want
    assert F.file_fingerprint(path, kind) == fingerprint
    parsed = F.read_header(path, kind)
    assert parsed["fingerprint"] == fingerprint
    offsets = [e["offset"] for e in parsed["tensors"]]
    assert offsets == sorted(offsets) and all(o % 64 == 0 for o in offsets)


def test_header_sections_follow_write_model_file(F):
    shapes = {"a": (2,)}
    header = json.loads(F.model_header({"x": 1}, shapes, {"licence": {"id": "mit"}, "edits": None}, ["a"]))
    assert header["tensors"] == [{"name": "a", "shape": [2], "dtype": "F32", "offset": 0, "nbytes": 8,
                                  "source_dtype": "F32"}]
    assert header["source"] is None and header["tokenizer"] is None and "edits" not in header
    assert header["fingerprint"] == "0" * 64


def test_writer_rejects_a_header_without_placeholder(F, tmp_path):
    with pytest.raises(ValueError, match="placeholder"):
        F.write_tensor_file(tmp_path / "x.dllm", 0, b'{"fingerprint":"abc"}', [np.ones(2, np.float32)])


# Files written by the reference's own write_model_file (tests/golden/make_model_file_goldens.py): the header bytes,
# fingerprint and whole-file hash for two architectures, with non-ASCII text, a float that needs 17 digits and the
# optional sections in the metadata.
MODEL_FILES = json.loads((Path(__file__).parent / "golden" / "model_file_header.json").read_text(encoding="utf-8"))


def golden_tensor_values(name: str, shape) -> np.ndarray:
    """The tensor values of those files: ((7 i + len(name)) mod 13 - 6) / 8 over the flat index i."""
    n = int(np.prod(shape)) if len(shape) else 1
    i = np.arange(n, dtype=np.int64)
    return (((7 * i + len(name)) % 13 - 6).astype(np.float32) / np.float32(8)).reshape(shape)


@pytest.mark.parametrize("case", sorted(MODEL_FILES))
def test_writer_matches_files_the_reference_wrote(F, tmp_path, case):
    import oracle_lib as O

    g = MODEL_FILES[case]
    order = O.tensor_order(g["shapes"])
    header = F.model_header(g["architecture"], g["shapes"], g["metadata"], order)
    path = tmp_path / "model.dllm"
    fingerprint = F.write_tensor_file(path, 0, header, [golden_tensor_values(n, g["shapes"][n]) for n in order])
    raw = path.read_bytes()
    length = struct.unpack_from("<Q", raw, 8)[0]
    assert raw[16:16 + length].decode("utf-8") == g["header"]
    assert fingerprint == g["fingerprint"] and F.file_fingerprint(path, F.MODEL) == g["fingerprint"]
    assert len(raw) == g["file_bytes"] and hashlib.sha256(raw).hexdigest() == g["file_sha256"]
