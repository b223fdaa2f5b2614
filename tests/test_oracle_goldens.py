"""The oracle against the reference's own golden values (tests/golden/reference_goldens.json, extracted from the
reference's tests/golden_values.py): random generator, forward kernel fingerprints, the gradient fingerprints of the
tiny fixture models and the 6-step fine-tuning fingerprints. These pin the C restatement of kernels and
orchestration end to end."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_goldens.json").read_text())
TOKENS = [1, 17, 42, 5, 63, 0, 9, 9, 30]  # reference tests/test_training.py:32
TARGETS = [*TOKENS[1:], 2]  # reference tests/test_training.py:50


def test_random_generator_matches_the_reference_goldens():
    r = O.Random(42)
    assert r.next_u64() == GOLDEN["RANDOM_FIRST"]
    assert r.next_u64() == GOLDEN["RANDOM_SECOND"]


def test_forward_kernel_fingerprints():
    """reference tests/test_kernels.py:331-350 for the kernels the training forward pass uses."""
    k = O.oracle_kernels()
    x, w = O.gaussian(20, 8, 64), O.gaussian(21, 48, 64)
    q, kk, v = O.gaussian(22, 8, 4, 16), O.gaussian(23, 8, 2, 16), O.gaussian(24, 8, 2, 16)
    outputs = {
        "linear": k.linear(x, w, O.gaussian(25, 48)),
        "rms_norm": k.rms_norm(x, O.gaussian(26, 64), 1e-6),
        "silu": k.silu(x),
        "rope": k.rope(q, np.arange(8, dtype=np.int64) * 97, O.rope_inv_freq(16, 10000.0)),
        "attention": k.attention(q, kk, v, 1.0 / np.sqrt(16.0)),
    }
    for name, values in outputs.items():
        assert O.tensor_fingerprint(values) == GOLDEN["KERNEL_FINGERPRINTS"][name], name


@pytest.mark.parametrize("family", sorted(O.FIXTURES))
def test_gradient_fingerprint(family):
    d = O.FIXTURES[family]
    _, _, grads = O.window_gradients(O.oracle_kernels(), d, O.fixture_weights(d), TOKENS, TARGETS)
    assert O.fingerprint(O.concatenated(grads)) == GOLDEN["GRADIENT_FINGERPRINT"][family]


def ascii_windows():
    """reference tests/test_training.py:310-312 (ascii_data, sequence length 8)."""
    documents = ["the quick brown fox jumps over the lazy dog", "pack my box with five dozen liquor jugs"]
    return O.windows_from_documents(documents, lambda text: [ord(c) % 64 for c in text], 8, 2)


@pytest.mark.parametrize("family", sorted(O.FIXTURES))
def test_finetune_fingerprint(family):
    """RUN = 6 steps, batch 3, sequence 8, seed 3, lr 1e-2, cosine (reference tests/test_training.py:357)."""
    d = O.FIXTURES[family]
    windows = ascii_windows()
    params = {n: a.copy() for n, a in O.fixture_weights(d).items()}
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=1e-2)
    losses = []
    for step in range(6):
        batch = [windows[i] for i in O.batch_indices(len(windows), step, 3, 3)]
        loss, _, _, _ = O.train_step(O.oracle_kernels(), d, params, m, v, batch, opt, step + 1, 6)
        losses.append(loss)
    assert O.data_fingerprint(params) == GOLDEN["FINETUNE_FINGERPRINT"][family]
    assert losses[-1] < losses[0]


LORA_FAMILIES = sorted(set(O.FIXTURES) & set(GOLDEN["LORA_FINETUNE_FINGERPRINT"]))


@pytest.mark.parametrize("family", LORA_FAMILIES)
def test_lora_finetune_fingerprint(family):
    """RUN = 6 steps, batch 3, sequence 8, seed 3, lr 3e-2 cosine, LoRA rank 2 alpha 4 on every target; the merged
    export's fingerprint (reference tests/test_lora.py:26-27,151-171)."""
    d = O.FIXTURES[family]
    lora = O.Lora(rank=2, alpha=4.0)
    kern = O.oracle_kernels()
    base = O.fixture_weights(d)
    adapters = O.init_adapters(d, lora, 3)
    m = {n: np.zeros_like(a) for n, a in adapters.items()}
    v = {n: np.zeros_like(a) for n, a in adapters.items()}
    windows = ascii_windows()
    opt = O.AdamWConfig(learning_rate=3e-2)
    for step in range(6):
        batch = [windows[i] for i in O.batch_indices(len(windows), step, 3, 3)]
        O.lora_train_step(kern, d, base, adapters, m, v, batch, opt, step + 1, 6, lora)
    merged = O.merged_weights(kern, d, base, adapters, lora)
    assert O.data_fingerprint(merged) == GOLDEN["LORA_FINETUNE_FINGERPRINT"][family]


# -- the router load-balancing loss: the reference pins it by formula and finite differences
#    (tests/test_moe_training.py:141-172); no golden holds it, so the oracle is pinned the same way.

@pytest.mark.parametrize("family", ["mixtral", "olmoe"])
def test_router_loss_gradient_matches_finite_differences(family):
    """Scale 0: only the load-balancing loss has a gradient (test_moe_training.py:151-172), through the router of
    the last layer and, via the routed mixture, a first-layer projection; the final norm gets none."""
    d = O.FIXTURES[family]
    weights = {n: a.copy() for n, a in O.fixture_weights(d).items()}
    kern = O.oracle_kernels()
    _, _, grads = O.window_gradients(kern, d, weights, TOKENS, TARGETS, scale=0.0, router_scale=1.0)
    rng = O.Random(3)
    for name in (f"layers.{d.layers - 1}.mlp.router.weight", "layers.0.attention.q.weight"):
        index = np.unravel_index(rng.next_u64() % weights[name].size, weights[name].shape)
        eps = 1e-2

        def at(delta, name=name, index=index):
            changed = dict(weights)
            changed[name] = weights[name].copy()
            changed[name][index] += np.float32(delta)
            return O.window_gradients(kern, d, changed, TOKENS, TARGETS, scale=0.0, router_scale=1.0)[1]

        numeric = (at(eps) - at(-eps)) / (2 * eps)
        assert float(grads[name][index]) == pytest.approx(numeric, rel=5e-2, abs=1e-4), name
    assert not np.any(grads["final_norm.weight"])


def test_router_loss_of_a_uniform_router_is_k():
    """Zero router weights: every probability is 1/E and every row picks experts 0..k-1 (ties to the lower index), so
    E * sum_e f_e * mean_e = E * k * (1/E) = k, and the gradient row is router_scale * E * f_e / T."""
    d = O.FIXTURES["mixtral"]
    weights = {n: (np.zeros_like(a) if n.endswith("router.weight") else a) for n, a in O.fixture_weights(d).items()}
    _, router_loss, _ = O.window_gradients(O.oracle_kernels(), d, weights, TOKENS, TARGETS, router_scale=0.0)
    assert router_loss == d.topk


def test_experts_no_token_reaches_get_zero_gradients():
    """test_moe_training.py:103-114: a one-token window routes to topk experts per layer; the others' gradients are
    exactly zero and the reached ones' are not."""
    d = O.FIXTURES["mixtral"]
    weights = O.fixture_weights(d)
    _, _, grads = O.window_gradients(O.oracle_kernels(), d, weights, [5], [7])
    for layer in range(d.layers):
        reached = [e for e in range(d.experts) if np.any(grads[f"layers.{layer}.mlp.experts.{e}.down.weight"])]
        assert len(reached) == d.topk
        for e in range(d.experts):
            for which in ("gate", "up", "down"):
                assert bool(np.any(grads[f"layers.{layer}.mlp.experts.{e}.{which}.weight"])) == (e in reached)


# The reference's DPO run (tests/test_preference.py:30-47, 223-244): five pairs, sequence length 24, end token 2,
# RunConfig(5, 2, 24, 3, AdamWConfig(learning_rate=1e-2), objective="dpo", beta=0.5).
DPO_RECORDS = [("the quick brown", " fox", " cat"), ("pack my box", " with jugs", " of"),
               ("two plus two is", " four", " five and a lot more words"), ("hello", " there", " go away"),
               ("the lazy", " dog", " frog")]
DPO_FAMILIES = sorted(set(O.FIXTURES) & set(GOLDEN["DPO_FINETUNE_FINGERPRINT"]))


def dpo_pairs():
    return O.preference_pairs(DPO_RECORDS, lambda text: [ord(c) % 64 for c in text], 24, 2)


@pytest.mark.parametrize("family", DPO_FAMILIES)
def test_oracle_reproduces_the_dpo_finetune_fingerprint(family):
    d = O.FIXTURES[family]
    kern = O.oracle_kernels()
    params = O.fixture_weights(d)
    pairs = dpo_pairs()
    reference = [(O.log_probability(kern, d, params, p, "chosen"), O.log_probability(kern, d, params, p, "rejected"))
                 for p in pairs]
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=1e-2)
    losses = []
    for step in range(5):
        batch = O.batch_indices(len(pairs), step, 2, 3)
        loss, _, _ = O.dpo_train_step(kern, d, params, m, v, [pairs[i] for i in batch],
                                      [reference[i] for i in batch], 0.5, opt, step + 1, 5)
        losses.append(loss)
    assert losses[0] == O.oracle().orc_log(2.0)  # the model is its own reference at step 1 (z = 0)
    assert O.data_fingerprint(params) == GOLDEN["DPO_FINETUNE_FINGERPRINT"][family]
