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


# ---- RoPE scaling (numerics.py:267-349) and the LongRoPE / YaRN attention factor (transformer.py:204-245) ----

PROMPT = [1, 17, 42, 5, 63, 0, 9, 9, 30]  # reference tests/test_transformer.py:17


def yarn_scaling(factor: float, original: int) -> dict:
    """importer.yarn_scaling (importing/importer.py:180-201) with its defaults: beta_fast 32, beta_slow 1, truncated,
    attention factor 0.1 ln(factor) + 1 in the portable log (_yarn_mscale, :176-177)."""
    return {"rope_type": "yarn", "factor": factor, "original_max_position_embeddings": original, "beta_fast": 32.0,
            "beta_slow": 1.0, "truncate": True,
            "attention_factor": 0.1 * 1.0 * O.oracle().orc_log(factor) + 1.0 if factor > 1.0 else 1.0}


@pytest.mark.parametrize("family", sorted(O.FIXTURES))
def test_forward_logits_match_tiny_logits_fingerprint(family):
    """The next-token logits of PROMPT on the tiny imported models (golden_values.py TINY_LOGITS_FINGERPRINT)."""
    d = O.FIXTURES[family]
    logits = O.logits(O.oracle_kernels(), d, O.fixture_weights(d), PROMPT)
    assert O.fingerprint(logits[-1]) == GOLDEN["TINY_LOGITS_FINGERPRINT"][family]


@pytest.mark.parametrize(("name", "family", "factor", "original"), [
    ("llama-yarn", "llama", 4.0, 2048),  # dllm import --context-length 8192 of the tiny Llama (2048 positions)
    ("qwen3-yarn", "qwen3", 4.0, 4),  # Qwen3 with a YaRN rope_scaling: the factor folds into its QK-norm weights
    ("olmo2-yarn", "olmo2", 2.0, 2048),  # --context-length 4096 of OLMo 2: folds into its whole-projection QK-norm
])
def test_yarn_models_match_long_context_fingerprints(name, family, factor, original):
    """reference tests/test_long_context.py:168-189 (LONG_MODELS): the YaRN frequencies and the attention factor
    folded into the q/k rows (or the QK-norm weights), through the whole forward pass, against the reference's
    LONG_CONTEXT_FINGERPRINTS."""
    from dataclasses import replace

    d = O.FIXTURES[family]
    scaling = yarn_scaling(factor, original)
    scaled = replace(d, inv_freq=tuple(O.rope_inv_freq_scaled(d.head_dim, d.rope_theta, scaling)),
                     rope_attention_factor=scaling["attention_factor"])
    logits = O.logits(O.oracle_kernels(), scaled, O.fixture_weights(d), PROMPT)
    assert O.fingerprint(logits[-1]) == GOLDEN["LONG_CONTEXT_FINGERPRINTS"][name]


def test_phi3_long_factors_match_the_long_context_fingerprint():
    """reference tests/test_long_context.py:113-118,160 ("phi3-long"): Phi-3 imported with a 1024-token context takes
    the LongRoPE long factors (factor_set "long"), the attention factor unchanged; its logits of PROMPT."""
    from dataclasses import replace

    d = O.FIXTURES["phi3"]
    long = replace(d, rope_scaling=O.frozen_scaling({**O.PHI3_SCALING, "factor_set": "long"}))
    assert long.c().rope_attention_factor == d.c().rope_attention_factor
    logits = O.logits(O.oracle_kernels(), long, O.fixture_weights(d), PROMPT)
    assert O.fingerprint(logits[-1]) == GOLDEN["LONG_CONTEXT_FINGERPRINTS"]["phi3-long"]


def test_rope_scaling_closed_forms():
    """reference tests/test_kernels.py:190-209 and test_long_context.py:29-50: linear and LongRoPE divide each default
    frequency by their factor (one correctly rounded division); llama3 keeps the short wavelengths, divides the long
    ones by the factor and interpolates strictly between in the band; YaRN follows transformers' float64 formula to
    1e-13, its fastest pair extrapolates and its slowest interpolates exactly; the default is theta^(-2i/d)."""
    plain = O.rope_inv_freq_scaled(64, 500000.0)
    np.testing.assert_allclose(plain, [500000.0 ** (-2 * i / 64) for i in range(32)], rtol=1e-14)
    assert plain.tobytes() == O.rope_inv_freq(64, 500000.0).tobytes()
    linear = O.rope_inv_freq_scaled(64, 500000.0, {"type": "linear", "factor": 4.0})
    assert linear.tobytes() == (plain / 4).tobytes()
    factors = [1.0 + 0.37 * i for i in range(16)]
    longrope = O.rope_inv_freq_scaled(32, 10000.0, {"rope_type": "longrope", "short_factor": factors,
                                                    "long_factor": [2.0] * 16})
    assert longrope.tobytes() == (O.rope_inv_freq_scaled(32, 10000.0) / np.array(factors)).tobytes()
    long = O.rope_inv_freq_scaled(32, 10000.0, {"rope_type": "longrope", "short_factor": factors,
                                                "long_factor": [2.0] * 16, "factor_set": "long"})
    assert long.tobytes() == (O.rope_inv_freq_scaled(32, 10000.0) / 2.0).tobytes()
    llama3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
              "original_max_position_embeddings": 8192}
    plain = O.rope_inv_freq_scaled(128, 500000.0)
    scaled = O.rope_inv_freq_scaled(128, 500000.0, llama3)
    assert scaled[0] == plain[0] and scaled[-1] == plain[-1] / 8
    band = [i for i, f in enumerate(plain) if 2048 < 2 * np.pi / f < 8192]
    assert band and all(plain[i] / 8 < scaled[i] < plain[i] for i in band)
    for scaling in ({"factor": 4.0, "original_max_position_embeddings": 32768},
                    {"factor": 2.5, "original_max_position_embeddings": 4096, "beta_fast": 16.0, "beta_slow": 2.0},
                    {"factor": 8.0, "original_max_position_embeddings": 2048, "truncate": False},
                    {"factor": 4.0, "original_max_position_embeddings": 64}):
        scaling = {"rope_type": "yarn", **scaling}
        ours = O.rope_inv_freq_scaled(128, 1_000_000.0, scaling)
        base = 1_000_000.0 ** (-np.arange(0, 128, 2, dtype=np.float64) / 128)

        def correction(rotations):
            return 128 * np.log(scaling["original_max_position_embeddings"] / (rotations * 2 * np.pi)) / (
                2 * np.log(1_000_000.0))

        low, high = correction(scaling.get("beta_fast", 32)), correction(scaling.get("beta_slow", 1))
        if scaling.get("truncate", True):
            low, high = np.floor(low), np.ceil(high)
        low, high = max(low, 0), min(high, 127)
        high = high + 0.001 if low == high else high
        extrapolation = 1 - np.clip((np.arange(64) - low) / (high - low), 0, 1)
        want = base / scaling["factor"] * (1 - extrapolation) + base * extrapolation
        np.testing.assert_allclose(ours, want, rtol=1e-13, atol=0)
        default = O.rope_inv_freq_scaled(128, 1_000_000.0)
        assert ours[0] == default[0] and ours[-1] == default[-1] / scaling["factor"]
    tiny = O.rope_inv_freq_scaled(8, 10000.0, {"rope_type": "yarn", "factor": 2.0,
                                               "original_max_position_embeddings": 1, "truncate": True})
    assert np.all(np.isfinite(tiny))


def test_attention_factor_fold_is_a_weight_scale():
    """The attention factor is fold_scales (transformer.py:224-245): the model with factor a equals the unscaled model
    on weights whose rotated q/k rows are multiplied by f32(a), and the gradients of the stored weights are those
    of the folded ones with the same rows times f32(a) (_unfold, backprop.py:380-394). Partial rotary: rows past
    rotary_dim in each head keep their values."""
    from dataclasses import replace

    d = replace(O.FIXTURES["qwen2"], rotary_dim=2)  # head_dim 4 (attention biases: the bias rows fold too)
    w = O.fixture_weights(d)
    a = 1.25
    folded = dict(w)
    hd, rd = d.head_dim, d.rotary_dim
    for name in w:
        if name.endswith(("attention.q.weight", "attention.q.bias", "attention.k.weight", "attention.k.bias")):
            rows = w[name].reshape(-1, hd, *w[name].shape[1:]).copy()
            rows[:, :rd] *= np.float32(a)
            folded[name] = rows.reshape(w[name].shape)
    scaled = replace(d, rope_attention_factor=a)
    kern = O.oracle_kernels()
    assert O.logits(kern, scaled, w, PROMPT).tobytes() == O.logits(kern, d, folded, PROMPT).tobytes()
    loss_a, _, g_a = O.window_gradients(kern, scaled, w, PROMPT[:-1], PROMPT[1:])
    loss_f, _, g_f = O.window_gradients(kern, d, folded, PROMPT[:-1], PROMPT[1:])
    assert loss_a == loss_f
    for name in w:
        want = g_f[name]
        if name in folded and folded[name] is not w[name]:
            rows = want.reshape(-1, hd, *want.shape[1:]).copy()
            rows[:, :rd] *= np.float32(a)
            want = rows.reshape(want.shape)
        assert g_a[name].tobytes() == want.tobytes(), name


# -- LoRA on a Q4_0 base (reference tests/test_quantized_finetuning.py:27-29,34-37,96-112): the tiny models with
#    hidden size 32 and vocabulary 264, every quantisable matrix replaced by its dequantised Q4_0 blocks.

QLORA_FIXTURES = O.QLORA_FIXTURES


def q4_0_base(d, weights):
    """lora.py:322-375 (dequantized_weights): q/k/v/o/gate/up/down matrices whose rows hold whole 32-value blocks
    become int8(unpacked Q4_0) * their block scale, elementwise in float32 (numerics.py:135-137)."""
    base = dict(weights)
    for name, shape in d.tensor_shapes().items():
        if O.quantizable(name, shape):
            packed, scales = O.quantize_q4_0(O.oracle().orc_quantize_q4_0, weights[name])
            values = O.unpack_q4_0(O.oracle().orc_unpack_q4_0, packed)
            base[name] = O.dequantize_q8_0(values, scales).reshape(shape)
    return base


def qlora_run(family, kern, on_step=None):
    """RUN = 4 steps, batch 2, sequence 8, seed 3, lr 3e-2 cosine, LoRA rank 2 alpha 4 on every target."""
    d = QLORA_FIXTURES[family]
    lora = O.Lora(rank=2, alpha=4.0)
    base = q4_0_base(d, O.fixture_weights(d))
    adapters = O.init_adapters(d, lora, 3)
    m = {n: np.zeros_like(a) for n, a in adapters.items()}
    v = {n: np.zeros_like(a) for n, a in adapters.items()}
    windows = ascii_windows()
    opt = O.AdamWConfig(learning_rate=3e-2)
    for step in range(4):
        batch = [windows[i] for i in O.batch_indices(len(windows), step, 2, 3)]
        O.lora_train_step(kern, d, base, adapters, m, v, batch, opt, step + 1, 4, lora)
    return d, lora, base, adapters


@pytest.mark.parametrize("family", sorted(QLORA_FIXTURES))
def test_qlora_finetune_fingerprint(family):
    """The merged export of the Q4_0-base run equals the reference's QLORA_FINETUNE_FINGERPRINT."""
    kern = O.oracle_kernels()
    d, lora, base, adapters = qlora_run(family, kern)
    merged = O.merged_weights(kern, d, base, adapters, lora)
    assert O.data_fingerprint(merged) == GOLDEN["QLORA_FINETUNE_FINGERPRINT"][family]
