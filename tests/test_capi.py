"""The C ABI without a GPU: the built library loads and exports every function include/dllm_hip.h declares, and the
host-side argument checks reject what the reference binding rejects before any device work."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dllm_hip.h"
LIBRARY = ROOT / "etalii_dllm_amd" / "libdllm_hip.so"

needs_library = pytest.mark.skipif(not LIBRARY.exists(), reason="libdllm_hip.so not built")


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(dllm_hip_\w+)\s*\(", text)))


def test_header_declares_the_hot_path_entry_points():
    names = set(declared_functions())
    for kernel in ("linear", "linear_backward", "rms_norm", "rms_norm_backward", "rope", "attention",
                   "attention_backward", "silu", "swiglu", "silu_backward", "cross_entropy", "embedding_backward",
                   "sum_squares", "adamw_step", "trainer_create", "trainer_step", "trainer_gradients"):
        assert f"dllm_hip_{kernel}" in names


@needs_library
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIBRARY))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing


@needs_library
def test_argument_errors_are_value_errors_without_touching_the_gpu():
    from etalii_dllm_amd import kernels

    with pytest.raises(ValueError, match="in_features"):
        kernels.linear(np.ones((2, 3), np.float32), np.ones((4, 5), np.float32))
    with pytest.raises(ValueError, match="multiple of kv heads"):
        kernels.attention(np.ones((2, 3, 4), np.float32), np.ones((2, 2, 4), np.float32),
                          np.ones((2, 2, 4), np.float32), 0.5)
    with pytest.raises(ValueError, match="head_dim"):
        kernels.rope(np.ones((2, 1, 4), np.float32), np.arange(2), np.ones(3))
    with pytest.raises(ValueError, match="one size"):
        kernels.adamw_step(np.ones(3, np.float32), np.ones(2, np.float32), np.ones(3, np.float32),
                           np.ones(3, np.float32), 1e-3, 0.9, 0.999, 1e-8, 0.0, 0.1, 0.1)


@needs_library
def test_natural_tensor_order_and_names_match_the_oracle_layout():
    """The trainer's tensor table is computed on the host; the same names and order as modelfile.tensor_order."""
    import oracle_lib as O
    from etalii_dllm_amd import trainer

    names = ["layers.10.mlp.up.weight", "layers.2.attention.q.weight", "final_norm.weight", "token_embedding.weight",
             "layers.2.attention.k.weight"]
    assert O.tensor_order(names) == ["final_norm.weight", "layers.2.attention.k.weight",
                                     "layers.2.attention.q.weight", "layers.10.mlp.up.weight",
                                     "token_embedding.weight"]
    assert trainer.DecoderConfig  # the structure is defined and matches the header's field count
    assert len(trainer.DecoderConfig._fields_) == 34


@needs_library
def test_library_random_inputs_match_the_oracle_and_the_reference_goldens():
    """dllm_hip_random_tokens / dllm_hip_fill_gaussian (host functions: no GPU) are Random (random.hpp) and
    fill_gaussian (kernels.cpp:206-218): the first two draws of Random(42) are the reference's RANDOM_FIRST and
    RANDOM_SECOND (checked modulo several vocabularies, the form the library returns them in), and the Gaussians equal
    the oracle's (and the compiled reference's where it is built) bit for bit, scaled by one float multiply."""
    import json

    import oracle_lib as O
    from etalii_dllm_amd.kernels import lib

    golden = json.loads((ROOT / "tests" / "golden" / "reference_goldens.json").read_text())
    first, second = golden["RANDOM_FIRST"], golden["RANDOM_SECOND"]
    for vocab in (2, 3, 151936, 49152, 50304, (1 << 61) - 1, (1 << 63) - 1):
        out = np.empty(2, np.int64)
        assert lib.dllm_hip_random_tokens(ctypes.c_uint64(42), out.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(2),
                                          ctypes.c_int64(vocab)) == 0
        assert out.tolist() == [first % vocab, second % vocab], vocab
    r = O.Random(7)
    want = np.array([r.next_u64() % 151936 for _ in range(1000)], np.int64)
    got = np.empty(1000, np.int64)
    lib.dllm_hip_random_tokens(ctypes.c_uint64(7), got.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(1000),
                               ctypes.c_int64(151936))
    assert np.array_equal(got, want)
    for seed, n in ((0, 1), (11000, 4099), (2**63 + 5, 777)):
        want = O.fill_gaussian(seed, n)
        for scale in (1.0, 0.02):
            got = np.empty(n, np.float32)
            assert lib.dllm_hip_fill_gaussian(ctypes.c_uint64(seed), got.ctypes.data_as(ctypes.c_void_p),
                                              ctypes.c_size_t(n), ctypes.c_float(scale)) == 0
            assert got.tobytes() == (want * np.float32(scale)).tobytes(), (seed, n, scale)
        if O.reference_available():
            ref = np.empty(n, np.float32)
            O.ref().ref_fill_gaussian(ctypes.c_uint64(seed), ref.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(n))
            assert ref.tobytes() == want.tobytes()


@needs_library
def test_layer_indices_outside_the_model_are_refused():
    """architecture.py:237-254 raises ValueError for dense_layers / sliding_window_layers outside the model; so does
    the trainer's configuration, and indices past 63 travel as per-layer flags."""
    from etalii_dllm_amd.trainer import Decoder

    base = dict(vocab=64, hidden=16, intermediate=24, layers=66, heads=2, kv_heads=1, head_dim=8, rms_norm_eps=1e-6,
                rope_theta=1e6, tie_embeddings=True, sliding_window=4, experts=4, experts_per_token=2)
    with pytest.raises(ValueError, match="dense_layers must be layer indices"):
        Decoder(**base, dense_layers=(66,)).native()
    with pytest.raises(ValueError, match="dense_layers must be layer indices"):
        Decoder(**base, dense_layers=(-1,)).native()
    with pytest.raises(ValueError, match="sliding_window_layers must be layer indices"):
        Decoder(**base, window_layers=(0, 70)).native()
    cfg = Decoder(**base, dense_layers=(1, 65), window_layers=(0, 64)).native()
    assert [cfg.dense_layer_flags[i] for i in range(66)] == [int(i in (1, 65)) for i in range(66)]
    assert [cfg.full_attention_layer_flags[i] for i in range(66)] == [int(i not in (0, 64)) for i in range(66)]
    assert cfg.dense_layers == 0 and cfg.full_attention_layers == 0
