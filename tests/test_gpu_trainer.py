"""GPU parity of the device-resident step: the reference's own whole-model goldens (GRADIENT_FINGERPRINT and the
6-step FINETUNE_FINGERPRINT for the dense tiny fixtures) and bit equality with the oracle's step on a larger
random model with ragged windows."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_goldens.json").read_text())
TOKENS = [1, 17, 42, 5, 63, 0, 9, 9, 30]
DENSE = ["llama", "mistral", "qwen2", "qwen3"]


def gpu_decoder(d: O.Decoder):
    from etalii_dllm_amd.trainer import Decoder

    return Decoder(d.vocab, d.hidden, d.inter, d.layers, d.heads, d.kv_heads, d.head_dim, d.eps, d.rope_theta,
                   d.tied, d.attn_bias, d.qk_norm, d.window)


def make_trainer(d: O.Decoder, weights, max_tokens=64, max_windows=8, max_window=32):
    from etalii_dllm_amd.trainer import Trainer

    t = Trainer(gpu_decoder(d), max_tokens, max_windows, max_window)
    assert t.names == O.tensor_order(d.tensor_shapes())
    t.load(weights)
    return t


@pytest.mark.parametrize("family", DENSE)
def test_gradient_fingerprint_on_gpu(family):
    d = O.FIXTURES[family]
    t = make_trainer(d, O.fixture_weights(d))
    loss = t.gradients([TOKENS + [2]], scale=1.0)
    grads = {n: t.get(n, d.tensor_shapes()[n], t.GRAD) for n in t.names}
    assert O.fingerprint(O.concatenated(grads)) == GOLDEN["GRADIENT_FINGERPRINT"][family]
    want_loss, _, _ = O.window_gradients(O.oracle_kernels(), d, O.fixture_weights(d), TOKENS, TOKENS[1:] + [2])
    assert loss == want_loss


def ascii_windows():
    documents = ["the quick brown fox jumps over the lazy dog", "pack my box with five dozen liquor jugs"]
    return O.windows_from_documents(documents, lambda text: [ord(c) % 64 for c in text], 8, 2)


@pytest.mark.parametrize("family", DENSE)
def test_finetune_fingerprint_on_gpu(family):
    d = O.FIXTURES[family]
    windows = ascii_windows()
    t = make_trainer(d, O.fixture_weights(d))
    opt = O.AdamWConfig(learning_rate=1e-2)
    for step in range(6):
        batch = [windows[i] for i in O.batch_indices(len(windows), step, 3, 3)]
        t.step(batch, opt.learning_rate_at(step + 1, 6), step + 1)
    params = {n: t.get(n, d.tensor_shapes()[n]) for n in t.names}
    assert O.data_fingerprint(params) == GOLDEN["FINETUNE_FINGERPRINT"][family]


def test_step_matches_the_oracle_on_ragged_windows():
    d = O.Decoder("qwen2", vocab=300, hidden=64, inter=160, layers=2, heads=4, kv_heads=2, head_dim=16, eps=1e-6,
                  rope_theta=1e6, tied=True, attn_bias=True)
    weights = O.synthetic_weights(d, seed=5, scale=0.05)
    rng = O.Random(9)
    lengths = [33, 2, 70, 17]
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in lengths]
    t = make_trainer(d, weights, max_tokens=256, max_windows=4, max_window=128)
    params = {n: a.copy() for n, a in weights.items()}
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=1e-3, schedule="constant")
    for step in (1, 2):
        loss_gpu, norm_gpu = t.step(windows, 1e-3, step)
        loss_cpu, _, norm_cpu, grads = O.train_step(O.oracle_kernels(), d, params, m, v, windows, opt, step, 2)
        assert loss_gpu == loss_cpu and norm_gpu == norm_cpu
        for name in t.names:
            shape = d.tensor_shapes()[name]
            assert t.get(name, shape, t.GRAD).tobytes() == grads[name].tobytes(), name
            assert t.get(name, shape).tobytes() == params[name].tobytes(), name
            assert t.get(name, shape, t.M).tobytes() == m[name].tobytes(), name
            assert t.get(name, shape, t.V).tobytes() == v[name].tobytes(), name
