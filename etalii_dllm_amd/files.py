"""model.dllm and .dllmckpt files from device-resident training state (src/etalii_dllm/modelfile.py:68-136,228-235
and training/trainer.py:477-630), over the C ABI of include/dllm_hip.h.

The headers are built here exactly as the reference builds them (canonical JSON of the same dictionaries); the
library writes the prefix, pads the header, streams the tensor data out of device memory and patches the SHA-256
fingerprint into the header, so a file has the same bytes as the reference's writer produces for the same run.
"""

from __future__ import annotations

import ctypes as C
import json
import math
import struct
from collections.abc import Mapping, Sequence
from pathlib import Path
from typing import Any

import numpy as np

from etalii_dllm_amd.kernels import check, lib

MODEL, CHECKPOINT = 0, 1
PLACEHOLDER = "0" * 64
_MODEL_PREFIX = struct.Struct("<4sIQ")  # modelfile.py:32
_CHECKPOINT_PREFIX = struct.Struct("<8sIQ")  # trainer.py:88

lib.dllm_hip_sha256.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_char_p]
lib.dllm_hip_write_tensor_file.argtypes = [C.c_char_p, C.c_int, C.c_char_p, C.c_size_t,
                                           C.POINTER(C.c_void_p), C.POINTER(C.c_int64), C.c_size_t, C.c_char_p]
lib.dllm_hip_tensor_file_fingerprint.argtypes = [C.c_char_p, C.c_int, C.c_char_p]
lib.dllm_hip_trainer_fingerprint.argtypes = [C.c_void_p, C.c_int, C.c_char_p, C.c_void_p]
lib.dllm_hip_trainer_write_file.argtypes = [C.c_void_p, C.c_int, C.c_char_p, C.c_char_p, C.c_size_t, C.c_char_p,
                                            C.c_void_p]
lib.dllm_hip_trainer_read_checkpoint.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_void_p]


class CheckpointError(ValueError):
    """The file is not a checkpoint of this run, or its data does not match its fingerprint (trainer.py:83-84)."""


def canonical_json(value: Any) -> bytes:
    """modelfile.canonical_json (modelfile.py:50-51)."""
    return json.dumps(value, sort_keys=True, ensure_ascii=False, separators=(",", ":"), allow_nan=False).encode()


def _pad(length: int) -> int:
    return -length % 64


def sha256(data: bytes | np.ndarray, impl: int = 0) -> str:
    """SHA-256 on the host (impl 0: fastest, 1: portable, 2: x86 SHA extensions when the CPU has them)."""
    buf = np.frombuffer(data, np.uint8) if isinstance(data, bytes) else np.ascontiguousarray(data).view(np.uint8)
    out = C.create_string_buffer(65)
    check(lib.dllm_hip_sha256(buf.ctypes.data if buf.size else None, buf.size, impl, out))
    return out.value.decode()


def model_header(architecture: Mapping[str, Any], shapes: Mapping[str, Sequence[int]], metadata: Mapping[str, Any],
                 order: Sequence[str]) -> bytes:
    """The header write_model_file writes before the fingerprint is known (modelfile.py:80-119): tensor entries in
    `order` (natural name order), the metadata sections, and the 64-zero fingerprint."""
    entries, offset = [], 0
    for name in order:
        shape = [int(d) for d in shapes[name]]
        nbytes = math.prod(shape) * 4
        entries.append({"name": name, "shape": shape, "dtype": "F32", "offset": offset, "nbytes": nbytes,
                        "source_dtype": "F32"})
        offset += nbytes + _pad(nbytes)
    header = {
        "format": "dllm",
        "format_version": 1,
        "architecture": dict(architecture),
        "tensors": entries,
        "fingerprint": PLACEHOLDER,
        **{key: metadata.get(key) for key in ("source", "licence", "tokenizer", "chat_template")},
    }
    for section in ("fine_tuning", "adapter", "edits", "embedding", "classifier", "merge", "lineage"):
        if metadata.get(section) is not None:
            header[section] = metadata[section]
    return canonical_json(header)


def checkpoint_header(*, architecture: Mapping[str, Any], run: Mapping[str, Any], step: int, losses: Sequence[float],
                      base_fingerprint: str, data_fingerprint: str, metadata: Mapping[str, Any],
                      shapes: Mapping[str, Sequence[int]], order: Sequence[str],
                      reference: Sequence[tuple[float, float]] | None = None) -> bytes:
    """FineTuner.save_checkpoint's header (trainer.py:534-558): "param/<name>" entries, then adam_m/<name> and
    adam_v/<name> per tensor, in `order`."""
    tensors = [f"param/{name}" for name in order]
    for name in order:
        tensors += [f"adam_m/{name}", f"adam_v/{name}"]
    entries, offset = [], 0
    for full in tensors:
        shape = [int(d) for d in shapes[full.split("/", 1)[1]]]
        nbytes = math.prod(shape) * 4
        entries.append({"name": full, "shape": shape, "offset": offset, "nbytes": nbytes})
        offset += nbytes + _pad(nbytes)
    header = {
        "format": "dllm-checkpoint",
        "format_version": 1,
        "architecture": dict(architecture),
        "run": dict(run),
        "step": int(step),
        "losses": [float(x) for x in losses],
        "base_fingerprint": base_fingerprint,
        "data_fingerprint": data_fingerprint,
        "metadata": dict(metadata),
        **({} if reference is None else {"reference": [[float(c).hex(), float(r).hex()] for c, r in reference]}),
        "tensors": entries,
        "fingerprint": PLACEHOLDER,
    }
    return canonical_json(header)


def write_tensor_file(path: str | Path, kind: int, header: bytes, tensors: Sequence[np.ndarray]) -> str:
    """A file from host arrays (float32), the library's writer; returns the fingerprint."""
    arrays = [np.ascontiguousarray(t, dtype=np.float32) for t in tensors]
    ptrs = (C.c_void_p * max(len(arrays), 1))(*[a.ctypes.data for a in arrays])
    numels = (C.c_int64 * max(len(arrays), 1))(*[a.size for a in arrays])
    out = C.create_string_buffer(65)
    check(lib.dllm_hip_write_tensor_file(str(path).encode(), kind, header, len(header), ptrs, numels, len(arrays),
                                         out))
    return out.value.decode()


def file_fingerprint(path: str | Path, kind: int) -> str:
    """The SHA-256 of a file's data section (ModelFile.verify's hash, modelfile.py:354-366)."""
    out = C.create_string_buffer(65)
    check(lib.dllm_hip_tensor_file_fingerprint(str(path).encode(), kind, out))
    return out.value.decode()


def read_header(path: str | Path, kind: int) -> dict[str, Any]:
    """The JSON header of a model or checkpoint file."""
    prefix = _MODEL_PREFIX if kind == MODEL else _CHECKPOINT_PREFIX
    magic = b"DLLM" if kind == MODEL else b"DLLMCKPT"
    with Path(path).open("rb") as stream:
        raw = stream.read(prefix.size)
        if len(raw) != prefix.size:
            raise CheckpointError(f"{path}: not a {'model' if kind == MODEL else 'checkpoint'} file")
        found, version, length = prefix.unpack(raw)
        if found != magic:
            raise CheckpointError(f"{path}: not a {'model' if kind == MODEL else 'checkpoint'} file")
        if version != 1:
            raise CheckpointError(f"{path}: unsupported format version {version}")
        try:
            return json.loads(stream.read(length).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as error:
            raise CheckpointError(f"{path}: header is not valid JSON") from error
