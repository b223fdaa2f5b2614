"""GPU parity of the device-resident step: the reference's own whole-model goldens (GRADIENT_FINGERPRINT, the
6-step FINETUNE_FINGERPRINT and LORA_FINETUNE_FINGERPRINT for the tiny dense and mixture-of-experts fixtures) and bit
equality with the oracle's step on larger random models with ragged windows."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_goldens.json").read_text())
TOKENS = [1, 17, 42, 5, 63, 0, 9, 9, 30]
FAMILIES = ["llama", "mistral", "qwen2", "qwen3", "mixtral", "olmoe", "phi3", "granite", "granitemoe", "qwen3_moe", "olmo2", "gemma3", "gemma2", "qwen2_moe", "granitemoeshared"]


def gpu_decoder(d: O.Decoder):
    from etalii_dllm_amd.trainer import Decoder

    return Decoder(d.vocab, d.hidden, d.inter, d.layers, d.heads, d.kv_heads, d.head_dim, d.eps, d.rope_theta,
                   d.tied, d.attn_bias, d.qk_norm, d.window, d.experts, d.topk, d.normalize, d.expert_inter,
                   rotary_dim=d.rotary_dim, rope_scaling=d.scaling(), embedding_multiplier=d.embedding_multiplier,
                   attention_multiplier=d.attention_multiplier, residual_multiplier=d.residual_multiplier,
                   logits_scaling=d.logits_scaling, dense_layers=d.dense_layers, norm_placement=d.norm_placement,
                   norm_unit_offset=d.unit_offset, activation=d.activation, window_layers=d.window_layers,
                   local_rope_theta=d.local_rope_theta, attention_softcap=d.attention_softcap,
                   logits_softcap=d.logits_softcap, shared_inter=d.shared_inter, shared_gate=d.shared_gate)


def make_trainer(d: O.Decoder, weights, max_tokens=64, max_windows=8, max_window=32):
    from etalii_dllm_amd.trainer import Trainer

    t = Trainer(gpu_decoder(d), max_tokens, max_windows, max_window)
    assert t.names == O.tensor_order(d.tensor_shapes())
    t.load(weights)
    return t


@pytest.mark.parametrize("family", FAMILIES)
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


@pytest.mark.parametrize("family", FAMILIES)
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
    assert t.fingerprint() == GOLDEN["FINETUNE_FINGERPRINT"][family]  # hashed from device memory


def checkpoint_fields(d: O.Decoder, step: int, losses):
    return {"architecture": {"family": d.family, "hidden": d.hidden, "layers": d.layers}, "run": {"steps": 6},
            "step": step, "losses": losses, "base_fingerprint": "b" * 64, "data_fingerprint": "d" * 64,
            "metadata": {"lineage": [{"step": "import"}]}}


@pytest.mark.parametrize("family", ["llama", "olmoe"])
def test_export_and_checkpoint_resume_on_gpu(family, tmp_path):
    """test_training.py:365-400 on the GPU: a run checkpointed at step 3 and resumed in a fresh trainer gives the
    same final checkpoint and the same exported model, whose fingerprint is the reference's FINETUNE_FINGERPRINT."""
    from etalii_dllm_amd import files

    d = O.FIXTURES[family]
    shapes = d.tensor_shapes()
    windows = ascii_windows()
    opt = O.AdamWConfig(learning_rate=1e-2)
    batches = [[windows[i] for i in O.batch_indices(len(windows), step, 3, 3)] for step in range(6)]
    first = make_trainer(d, O.fixture_weights(d))
    losses = []
    for step in range(3):
        losses.append(first.step(batches[step], opt.learning_rate_at(step + 1, 6), step + 1)[0])
    middle = first.save_checkpoint(tmp_path / "middle.dllmckpt", shapes, **checkpoint_fields(d, 3, losses))
    assert middle == first.fingerprint(files.CHECKPOINT)
    for step in range(3, 6):
        losses.append(first.step(batches[step], opt.learning_rate_at(step + 1, 6), step + 1)[0])
    final = first.save_checkpoint(tmp_path / "final.dllmckpt", shapes, **checkpoint_fields(d, 6, losses))
    metadata = {"licence": {"id": "apache-2.0"}, "fine_tuning": {"steps_completed": 6, "final_loss": losses[-1]}}
    arch = {"family": d.family, "hidden": d.hidden}
    exported = first.export(tmp_path / "first.dllm", arch, metadata, shapes)
    assert exported == GOLDEN["FINETUNE_FINGERPRINT"][family]
    assert files.file_fingerprint(tmp_path / "first.dllm", files.MODEL) == exported
    header = files.read_header(tmp_path / "first.dllm", files.MODEL)
    assert [e["name"] for e in header["tensors"]] == O.tensor_order(shapes) and header["fingerprint"] == exported

    second = make_trainer(d, {n: np.zeros(s, np.float32) for n, s in shapes.items()})
    restored = second.load_checkpoint(tmp_path / "middle.dllmckpt", data_fingerprint="d" * 64)
    assert restored["step"] == 3 and restored["losses"] == losses[:3]
    for step in range(3, 6):
        assert second.step(batches[step], opt.learning_rate_at(step + 1, 6), step + 1)[0] == losses[step]
    assert second.save_checkpoint(tmp_path / "resumed.dllmckpt", shapes, **checkpoint_fields(d, 6, losses)) == final
    assert (tmp_path / "resumed.dllmckpt").read_bytes() == (tmp_path / "final.dllmckpt").read_bytes()
    assert second.export(tmp_path / "second.dllm", arch, metadata, shapes) == exported
    assert (tmp_path / "second.dllm").read_bytes() == (tmp_path / "first.dllm").read_bytes()

    with pytest.raises(files.CheckpointError, match="different data"):
        second.load_checkpoint(tmp_path / "middle.dllmckpt", data_fingerprint="e" * 64)
    raw = bytearray((tmp_path / "middle.dllmckpt").read_bytes())
    raw[-1] ^= 1
    (tmp_path / "corrupt.dllmckpt").write_bytes(bytes(raw))
    with pytest.raises(files.CheckpointError, match="fingerprint"):
        second.load_checkpoint(tmp_path / "corrupt.dllmckpt")
    assert second.fingerprint(files.CHECKPOINT) == final  # a rejected file leaves the state alone


MODEL_FILES = json.loads((Path(__file__).parent / "golden" / "model_file_header.json").read_text(encoding="utf-8"))
EXPORT_DECODERS = {
    "llama_tied": O.Decoder("llama", vocab=64, hidden=16, inter=32, layers=2, heads=4, kv_heads=2, head_dim=4,
                            eps=1e-5, rope_theta=1e5, tied=True),
    "moe_post_norms": O.Decoder("olmoe", vocab=48, hidden=8, inter=12, layers=2, heads=2, kv_heads=1, head_dim=4,
                                eps=1e-6, rope_theta=1e4, tied=False, qk_norm=2, norm_placement=1, experts=4, topk=2,
                                normalize=False, expert_inter=6),
}


@pytest.mark.parametrize("case", sorted(EXPORT_DECODERS))
def test_export_matches_files_the_reference_wrote(case, tmp_path):
    """The trainer's export from device memory against model files the reference's own write_model_file wrote
    (tests/golden/make_model_file_goldens.py): the same bytes, header included."""
    import hashlib

    from test_files import golden_tensor_values

    d, g = EXPORT_DECODERS[case], MODEL_FILES[case]
    shapes = d.tensor_shapes()
    assert {n: list(s) for n, s in shapes.items()} == g["shapes"]
    t = make_trainer(d, {n: golden_tensor_values(n, s) for n, s in shapes.items()})
    fingerprint = t.export(tmp_path / "model.dllm", g["architecture"], g["metadata"], shapes)
    raw = (tmp_path / "model.dllm").read_bytes()
    assert fingerprint == g["fingerprint"]
    assert len(raw) == g["file_bytes"] and hashlib.sha256(raw).hexdigest() == g["file_sha256"]
    t.close()


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


def make_lora_trainer(d: O.Decoder, weights, lora: O.Lora, adapters, base_quantize=None, max_tokens=64,
                      max_windows=8, max_window=32):
    from etalii_dllm_amd.trainer import Trainer, lora_config

    t = Trainer(gpu_decoder(d), max_tokens, max_windows, max_window,
                lora=lora_config(lora.rank, lora.alpha, lora.targets, lora.rslora, base_quantize))
    assert t.names == O.tensor_order(d.tensor_shapes()) + O.tensor_order(O.adapter_shapes(d, lora))
    t.load(weights)
    t.load(adapters)
    return t


@pytest.mark.parametrize("family", [f for f in FAMILIES if f in GOLDEN["LORA_FINETUNE_FINGERPRINT"]])
def test_lora_finetune_fingerprint_on_gpu(family):
    """The reference's LoRA run (tests/test_lora.py:26-27,151-171) on the GPU; the merged export through the GPU
    merge."""
    from etalii_dllm_amd import kernels as K

    d = O.FIXTURES[family]
    lora = O.Lora(rank=2, alpha=4.0)
    base = O.fixture_weights(d)
    shapes = O.adapter_shapes(d, lora)
    t = make_lora_trainer(d, base, lora, O.init_adapters(d, lora, 3))
    windows = ascii_windows()
    opt = O.AdamWConfig(learning_rate=3e-2)
    for step in range(6):
        batch = [windows[i] for i in O.batch_indices(len(windows), step, 3, 3)]
        t.step(batch, opt.learning_rate_at(step + 1, 6), step + 1)
    adapters = {n: t.get(n, shapes[n]) for n in shapes}
    merged = dict(base)
    for name in O.lora_target_weights(d, lora):
        merged[name] = K.lora_merge(base[name], adapters[name + ".lora_a"], adapters[name + ".lora_b"], lora.scale)
    assert O.data_fingerprint(merged) == GOLDEN["LORA_FINETUNE_FINGERPRINT"][family]
    assert t.fingerprint() == GOLDEN["LORA_FINETUNE_FINGERPRINT"][family]  # merged on and hashed from the device


@pytest.mark.parametrize("family", sorted(O.QLORA_FIXTURES))
def test_qlora_finetune_fingerprint_on_gpu(family):
    """LoRA on a Q4_0 base (tests/test_quantized_finetuning.py:27-29,96-112): 4 steps, batch 2, seed 3, lr 3e-2,
    rank 2 alpha 4 on every target of the hidden-32 models; the GPU quantises and dequantises the base itself, and
    the merged export is the reference's QLORA_FINETUNE_FINGERPRINT."""
    d = O.QLORA_FIXTURES[family]
    lora = O.Lora(rank=2, alpha=4.0)
    t = make_lora_trainer(d, O.fixture_weights(d), lora, O.init_adapters(d, lora, 3), "q4_0")
    windows = ascii_windows()
    opt = O.AdamWConfig(learning_rate=3e-2)
    for step in range(4):
        batch = [windows[i] for i in O.batch_indices(len(windows), step, 2, 3)]
        t.step(batch, opt.learning_rate_at(step + 1, 4), step + 1)
    assert t.fingerprint() == GOLDEN["QLORA_FINETUNE_FINGERPRINT"][family]


def test_lora_checkpoint_holds_the_adapters_and_restores_the_run(tmp_path):
    """A LoRA checkpoint holds the adapters and their moments only (trainer.py:519-522, 616-622); restored into a
    trainer on the same base, the export is the reference's LORA_FINETUNE_FINGERPRINT."""
    from etalii_dllm_amd import files

    d = O.FIXTURES["llama"]
    lora = O.Lora(rank=2, alpha=4.0)
    base = O.fixture_weights(d)
    shapes = {**d.tensor_shapes(), **O.adapter_shapes(d, lora)}
    t = make_lora_trainer(d, base, lora, O.init_adapters(d, lora, 3))
    windows = ascii_windows()
    opt = O.AdamWConfig(learning_rate=3e-2)
    for step in range(6):
        batch = [windows[i] for i in O.batch_indices(len(windows), step, 3, 3)]
        t.step(batch, opt.learning_rate_at(step + 1, 6), step + 1)
    fields = checkpoint_fields(d, 6, [])
    saved = t.save_checkpoint(tmp_path / "lora.dllmckpt", shapes, **fields)
    header = files.read_header(tmp_path / "lora.dllmckpt", files.CHECKPOINT)
    assert all(e["name"].endswith((".lora_a", ".lora_b")) for e in header["tensors"])
    fresh = make_lora_trainer(d, base, lora, {n: np.zeros(s, np.float32) for n, s in O.adapter_shapes(d, lora).items()})
    fresh.load_checkpoint(tmp_path / "lora.dllmckpt")
    assert fresh.fingerprint(files.CHECKPOINT) == saved
    assert fresh.fingerprint() == GOLDEN["LORA_FINETUNE_FINGERPRINT"]["llama"]


@pytest.mark.parametrize("base_quantize", [None, "q8_0"])
def test_lora_step_matches_the_oracle_on_ragged_windows(base_quantize):
    """LoRA (rank 16, attention and MLP targets) on a float or Q8_0 base; the Q8_0 run against the oracle's LoRA on
    the dequantised base (test_quantized_finetuning.py:96-106: a quantised run is LoRA on the dequantised base)."""
    d = O.Decoder("qwen2", vocab=300, hidden=64, inter=160, layers=2, heads=4, kv_heads=2, head_dim=16, eps=1e-6,
                  rope_theta=1e6, tied=True, attn_bias=True)
    weights = O.synthetic_weights(d, seed=5, scale=0.05)
    lora = O.Lora(rank=16, alpha=32.0, targets=("q", "v", "o", "gate", "down"))
    adapters = O.init_adapters(d, lora, 7)
    for name in adapters:  # non-zero B so the merge and both adapter gradients are exercised
        if name.endswith(".lora_b"):
            adapters[name] = O.gaussian(len(name), *adapters[name].shape, scale=0.02)
    base = dict(weights)
    if base_quantize:
        for name, shape in d.tensor_shapes().items():
            if name.endswith((".q.weight", ".k.weight", ".v.weight", ".o.weight", ".gate.weight", ".up.weight",
                              ".down.weight")) and len(shape) == 2 and shape[1] % 32 == 0:
                q, s = O.quantize_q8_0(O.oracle().orc_quantize_q8_0, weights[name])
                base[name] = O.dequantize_q8_0(q, s).reshape(shape)
    rng = O.Random(9)
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in (33, 2, 70, 17)]
    t = make_lora_trainer(d, weights, lora, adapters, base_quantize, max_tokens=256, max_windows=4, max_window=128)
    kern = O.oracle_kernels()
    params = {n: a.copy() for n, a in adapters.items()}
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=1e-3, schedule="constant")
    for step in (1, 2):
        loss_gpu, norm_gpu = t.step(windows, 1e-3, step)
        loss_cpu, norm_cpu = O.lora_train_step(kern, d, base, params, m, v, windows, opt, step, 2, lora)
        assert loss_gpu == loss_cpu and norm_gpu == norm_cpu
        for name, a in params.items():
            assert t.get(name, a.shape).tobytes() == a.tobytes(), name
            assert t.get(name, a.shape, t.M).tobytes() == m[name].tobytes(), name
            assert t.get(name, a.shape, t.V).tobytes() == v[name].tobytes(), name
    # only the adapted weights' gradients are computed; the others reach no optimizer and stay zero
    for name in ("token_embedding.weight", "layers.0.attention.k.weight", "layers.1.mlp_norm.weight",
                 "layers.0.attention.q.bias", "final_norm.weight"):
        assert not np.any(t.get(name, d.tensor_shapes()[name], t.GRAD)), name
    assert np.any(t.get("layers.1.attention.v.weight", d.tensor_shapes()["layers.1.attention.v.weight"], t.GRAD))


MOE = {
    "mixtral": O.Decoder("mixtral", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=2, head_dim=16,
                         eps=1e-5, rope_theta=1e6, tied=False, experts=8, topk=2, normalize=True, expert_inter=48),
    "olmoe": O.Decoder("olmoe", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=4, head_dim=16,
                       eps=1e-5, rope_theta=1e4, tied=False, qk_norm=2, experts=16, topk=4, normalize=False,
                       expert_inter=32),
    # a dense first layer among routed ones (mlp_only_layers), per-head QK-norm
    "qwen3_moe": O.Decoder("qwen3_moe", vocab=256, hidden=64, inter=96, layers=3, heads=4, kv_heads=2, head_dim=16,
                           eps=1e-6, rope_theta=1e6, tied=True, qk_norm=1, experts=8, topk=2, normalize=True,
                           expert_inter=32, dense_layers=(0,)),
    # Granite's multipliers with routed experts: every expert's down projection folds the residual multiplier
    "granitemoe": O.Decoder("granitemoe", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=2, head_dim=16,
                            eps=1e-6, rope_theta=1e4, tied=True, experts=8, topk=2, normalize=True, expert_inter=32,
                            embedding_multiplier=12.0, attention_multiplier=0.0625, residual_multiplier=0.22,
                            logits_scaling=6.0),
    # a gated shared expert beside the routed ones, q/k/v biases
    "qwen2_moe": O.Decoder("qwen2_moe", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=2, head_dim=16,
                           eps=1e-6, rope_theta=1e6, tied=False, attn_bias=True, experts=8, topk=2, normalize=False,
                           expert_inter=32, shared_inter=48, shared_gate=True),
}


@pytest.mark.parametrize("family", sorted(MOE))
def test_moe_step_matches_the_oracle_on_ragged_windows(family):
    """Routed experts with the load-balancing loss (router_aux_loss 0.05): two steps over windows of 33, 2, 70 and
    17 tokens (the 1-row window reaches only topk experts, so most experts get a window of no rows), every gradient,
    parameter and moment against the oracle; then a 1-row batch in which most experts get no row at all
    (backprop.py:339-341: their gradients are zero)."""
    d = MOE[family]
    weights = O.synthetic_weights(d, seed=11, scale=0.05)
    rng = O.Random(21)
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in (33, 2, 70, 17)]
    t = make_trainer(d, weights, max_tokens=256, max_windows=4, max_window=128)
    params = {n: a.copy() for n, a in weights.items()}
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=1e-3, schedule="constant")
    for step in (1, 2):
        loss_gpu, norm_gpu = t.step(windows, 1e-3, step, router_aux_loss=0.05)
        loss_cpu, _, norm_cpu, grads = O.train_step(O.oracle_kernels(), d, params, m, v, windows, opt, step, 2,
                                                    router_aux_loss=0.05)
        assert loss_gpu == loss_cpu and norm_gpu == norm_cpu
        for name in t.names:
            shape = d.tensor_shapes()[name]
            assert t.get(name, shape, t.GRAD).tobytes() == grads[name].tobytes(), name
            assert t.get(name, shape).tobytes() == params[name].tobytes(), name
            assert t.get(name, shape, t.M).tobytes() == m[name].tobytes(), name
            assert t.get(name, shape, t.V).tobytes() == v[name].tobytes(), name
    window = windows[0][:2]
    loss = t.gradients([window], scale=0.5, router_scale=0.25)
    want_loss, want_router, want = O.window_gradients(O.oracle_kernels(), d, params, window[:1], window[1:],
                                                      scale=0.5, router_scale=0.25)
    assert loss == want_loss and t.router_loss() == want_router
    unreached = 0
    for name in t.names:
        got = t.get(name, d.tensor_shapes()[name], t.GRAD)
        assert got.tobytes() == want[name].tobytes(), name
        unreached += ".experts." in name and not np.any(got)
    assert unreached >= 3 * (d.experts - d.topk) * sum(d.is_sparse(layer) for layer in range(d.layers))


def test_moe_lora_step_matches_the_oracle():
    """LoRA on a routed model: gate/up/down adapt every expert's projection, the router is never adapted
    (lora.py:211-242); two steps against the oracle's LoRA step."""
    d = MOE["mixtral"]
    weights = O.synthetic_weights(d, seed=12, scale=0.05)
    lora = O.Lora(rank=4, alpha=8.0, targets=("q", "o", "gate", "down"))
    adapters = O.init_adapters(d, lora, 5)
    for name in adapters:
        if name.endswith(".lora_b"):
            adapters[name] = O.gaussian(len(name) + 1, *adapters[name].shape, scale=0.02)
    rng = O.Random(23)
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in (20, 41, 3)]
    t = make_lora_trainer(d, weights, lora, adapters, max_tokens=128, max_windows=4, max_window=64)
    state = {n: a.copy() for n, a in adapters.items()}
    m = {n: np.zeros_like(a) for n, a in state.items()}
    v = {n: np.zeros_like(a) for n, a in state.items()}
    opt = O.AdamWConfig(learning_rate=1e-3, schedule="constant")
    for step in (1, 2):
        loss_gpu, norm_gpu = t.step(windows, 1e-3, step, router_aux_loss=0.1)
        loss_cpu, norm_cpu = O.lora_train_step(O.oracle_kernels(), d, weights, state, m, v, windows, opt, step, 2,
                                               lora, router_aux_loss=0.1)
        assert loss_gpu == loss_cpu and norm_gpu == norm_cpu
        for name, value in state.items():
            assert t.get(name, value.shape).tobytes() == value.tobytes(), name


@pytest.mark.parametrize("window", [0, 100])
def test_attention_at_head_dim_128_matches_the_oracle(window):
    """The attention matmuls at their real tile shapes (head_dim 128: two 64-column tiles per lane; several 64-row
    tiles; grouped heads), causal and sliding-window, on windows of 300, 129 and 64 tokens: every gradient of one
    gradients() call against the oracle."""
    d = O.Decoder("mistral", vocab=256, hidden=128, inter=128, layers=1, heads=4, kv_heads=2, head_dim=128,
                  eps=1e-5, rope_theta=1e4, tied=False, window=window)
    weights = O.synthetic_weights(d, seed=31, scale=0.05)
    rng = O.Random(37)
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in (301, 130, 65)]
    t = make_trainer(d, weights, max_tokens=512, max_windows=4, max_window=320)
    scale = 1.0 / sum(len(w) - 1 for w in windows)
    loss = t.gradients(windows, scale=scale)
    kern = O.oracle_kernels()
    want_loss, want = 0.0, {}
    for w in windows:
        l, _, g = O.window_gradients(kern, d, weights, w[:-1], w[1:], scale=scale)
        want_loss += l
        for name, value in g.items():
            want[name] = want[name] + value if name in want else value.copy()
    assert loss == want_loss
    for name in t.names:
        assert t.get(name, d.tensor_shapes()[name], t.GRAD).tobytes() == want[name].tobytes(), name


@pytest.mark.parametrize("window", [0, 1000])
def test_windows_past_2048_tokens_match_the_oracle(window):
    """Windows of 2600 and 300 tokens (the step has no window-length cap; the reference has none): scores, softmax
    chains and the multiply-add tiles past 2048 keys per query, causal and with a sliding window, every gradient of
    one gradients() call against the oracle."""
    d = O.Decoder("mistral", vocab=128, hidden=64, inter=64, layers=1, heads=2, kv_heads=1, head_dim=32, eps=1e-5,
                  rope_theta=1e4, tied=False, window=window)
    weights = O.synthetic_weights(d, seed=41, scale=0.05)
    rng = O.Random(43)
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in (2601, 301)]
    t = make_trainer(d, weights, max_tokens=2900, max_windows=2, max_window=2600)
    scale = 1.0 / sum(len(w) - 1 for w in windows)
    loss = t.gradients(windows, scale=scale)
    kern = O.oracle_kernels()
    want_loss, want = 0.0, {}
    for w in windows:
        l, _, g = O.window_gradients(kern, d, weights, w[:-1], w[1:], scale=scale)
        want_loss += l
        for name, value in g.items():
            want[name] = want[name] + value if name in want else value.copy()
    assert loss == want_loss
    for name in t.names:
        assert t.get(name, d.tensor_shapes()[name], t.GRAD).tobytes() == want[name].tobytes(), name


DPO_RECORDS = [("the quick brown", " fox", " cat"), ("pack my box", " with jugs", " of"),
               ("two plus two is", " four", " five and a lot more words"), ("hello", " there", " go away"),
               ("the lazy", " dog", " frog")]


@pytest.mark.parametrize("family", [f for f in FAMILIES if f in GOLDEN["DPO_FINETUNE_FINGERPRINT"]])
def test_dpo_finetune_fingerprint_on_gpu(family):
    """The reference's DPO run (tests/test_preference.py:30-47, 223-244) on the GPU: the reference log-probabilities
    from the initial weights, five steps of two pairs, the loss log 2 at the first step, the export fingerprint."""
    d = O.FIXTURES[family]
    pairs = O.preference_pairs(DPO_RECORDS, lambda text: [ord(c) % 64 for c in text], 24, 2)
    t = make_trainer(d, O.fixture_weights(d), max_tokens=128, max_windows=4, max_window=32)
    reference = t.log_probabilities(pairs)
    kern = O.oracle_kernels()
    want = [(O.log_probability(kern, d, O.fixture_weights(d), p, "chosen"),
             O.log_probability(kern, d, O.fixture_weights(d), p, "rejected")) for p in pairs]
    assert reference == want
    opt = O.AdamWConfig(learning_rate=1e-2)
    losses = []
    for step in range(5):
        batch = O.batch_indices(len(pairs), step, 2, 3)
        losses.append(t.dpo_step([pairs[i] for i in batch], [reference[i] for i in batch], 0.5,
                                 opt.learning_rate_at(step + 1, 5), step + 1)[0])
    assert losses[0] == O.oracle().orc_log(2.0)
    assert t.fingerprint() == GOLDEN["DPO_FINETUNE_FINGERPRINT"][family]


def test_dpo_step_matches_the_oracle_on_ragged_pairs():
    """A DPO step on a larger random model with prompts and answers of uneven lengths: loss, norm, gradients,
    parameters and moments bit-equal to the oracle's (trainer.py:364-384)."""
    d = O.Decoder("qwen2", vocab=300, hidden=64, inter=160, layers=2, heads=4, kv_heads=2, head_dim=16, eps=1e-6,
                  rope_theta=1e6, tied=True, attn_bias=True)
    weights = O.synthetic_weights(d, seed=7, scale=0.05)
    rng = O.Random(11)
    shapes = [(5, 9, 3), (1, 40, 17), (23, 2, 30)]
    pairs = [(tuple(rng.next_u64() % d.vocab for _ in range(p)), tuple(rng.next_u64() % d.vocab for _ in range(c)),
              tuple(rng.next_u64() % d.vocab for _ in range(r))) for p, c, r in shapes]
    reference = [(-3.25, -4.5), (-61.0, -20.0), (-7.0, -80.0)]
    t = make_trainer(d, weights, max_tokens=256, max_windows=6, max_window=64)
    params = {n: a.copy() for n, a in weights.items()}
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=1e-3, schedule="constant")
    for step in (1, 2):
        loss_gpu, norm_gpu = t.dpo_step(pairs, reference, 0.3, 1e-3, step)
        loss_cpu, norm_cpu, grads = O.dpo_train_step(O.oracle_kernels(), d, params, m, v, pairs, reference, 0.3, opt,
                                                     step, 2)
        assert loss_gpu == loss_cpu and norm_gpu == norm_cpu
        for name in t.names:
            shape = d.tensor_shapes()[name]
            assert t.get(name, shape, t.GRAD).tobytes() == grads[name].tobytes(), name
            assert t.get(name, shape).tobytes() == params[name].tobytes(), name
            assert t.get(name, shape, t.M).tobytes() == m[name].tobytes(), name
            assert t.get(name, shape, t.V).tobytes() == v[name].tobytes(), name


ROPE_CASES = {
    # Phi-3-style: partial rotary (8 of 16 dimensions) with LongRoPE short factors and its attention factor, q/k biases
    "longrope-partial": (O.Decoder("qwen2", vocab=300, hidden=64, inter=96, layers=2, heads=4, kv_heads=2,
                                   head_dim=16, eps=1e-6, rope_theta=1e4, tied=False, attn_bias=True, rotary_dim=8),
                         {"rope_type": "longrope", "short_factor": [1.0, 1.5, 3.25, 7.0],
                          "long_factor": [2.0, 3.0, 4.0, 5.0], "attention_factor": 1.1902380714238083}, None),
    # Qwen3 with YaRN: the factor folds into the per-head QK-norm weights
    "yarn-qk-norm": (O.Decoder("qwen3", vocab=256, hidden=64, inter=128, layers=2, heads=4, kv_heads=2, head_dim=16,
                               eps=1e-6, rope_theta=1e6, tied=True, qk_norm=1),
                     {"rope_type": "yarn", "factor": 4.0, "original_max_position_embeddings": 64, "beta_fast": 32.0,
                      "beta_slow": 1.0, "truncate": True, "attention_factor": 1.1386294361119891}, None),
    # llama3 frequencies (no attention factor) with partial rotary, whole-projection QK-norm and routed experts
    "llama3-olmoe": (O.Decoder("olmoe", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=4, head_dim=16,
                               eps=1e-5, rope_theta=5e5, tied=False, qk_norm=2, experts=8, topk=2, normalize=False,
                               expert_inter=32, rotary_dim=12),
                     {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                      "original_max_position_embeddings": 64}, None),
    # LoRA on q and k of a YaRN model: the factor folds into the merged weights
    "yarn-lora": (O.Decoder("llama", vocab=300, hidden=64, inter=96, layers=2, heads=4, kv_heads=2, head_dim=16,
                            eps=1e-5, rope_theta=1e5, tied=True),
                  {"rope_type": "yarn", "factor": 2.0, "original_max_position_embeddings": 32, "beta_fast": 32.0,
                   "beta_slow": 1.0, "truncate": True, "attention_factor": 1.0693147180559945},
                  O.Lora(rank=4, alpha=8.0, targets=("q", "k", "o"))),
}


@pytest.mark.parametrize("case", sorted(ROPE_CASES))
def test_step_with_rope_scaling_matches_the_oracle(case):
    """RoPE scaling in the trainer (numerics.py:267-349): the scaled inverse frequencies (LongRoPE short factors,
    YaRN, llama3), partial rotary, and the LongRoPE / YaRN attention factor folded into the q/k rows or the QK-norm
    weights (transformer.py:204-245) with the per-window gradient unfold (backprop.py:380-394); two steps over ragged
    windows against the oracle, every gradient, parameter and moment (adapters and their moments for LoRA)."""
    from dataclasses import replace

    from etalii_dllm_amd import kernels as K
    from etalii_dllm_amd.trainer import Decoder, Trainer, lora_config

    d, scaling, lora = ROPE_CASES[case]
    inv = K.rope_inv_freq(d.head_dim, d.rope_theta, rotary_dim=d.rotary_dim or None, scaling=scaling)
    assert inv.tobytes() == O.rope_inv_freq_scaled(d.rotary_dim or d.head_dim, d.rope_theta, scaling).tobytes()
    od = replace(d, inv_freq=tuple(inv), rope_attention_factor=K.rope_attention_factor(scaling))
    weights = O.synthetic_weights(d, seed=31, scale=0.05)
    rng = O.Random(33)
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in (33, 2, 70, 17)]
    gd = Decoder(d.vocab, d.hidden, d.inter, d.layers, d.heads, d.kv_heads, d.head_dim, d.eps, d.rope_theta, d.tied,
                 d.attn_bias, d.qk_norm, d.window, d.experts, d.topk, d.normalize, d.expert_inter,
                 rotary_dim=d.rotary_dim, rope_scaling=scaling)
    opt = O.AdamWConfig(learning_rate=1e-3, schedule="constant")
    if lora is None:
        t = Trainer(gd, 256, 4, 128)
        t.load(weights)
        params = {n: a.copy() for n, a in weights.items()}
        m = {n: np.zeros_like(a) for n, a in params.items()}
        v = {n: np.zeros_like(a) for n, a in params.items()}
        # the parameters are read back only after the last step (reading them marks them as written, which would
        # rebuild the folded copies before the next step whatever the step itself keeps up to date)
        for step in (1, 2, 3):
            loss_gpu, norm_gpu = t.step(windows, 1e-3, step, router_aux_loss=0.02 if d.experts else 0.0)
            loss_cpu, _, norm_cpu, grads = O.train_step(O.oracle_kernels(), od, params, m, v, windows, opt, step, 3,
                                                        router_aux_loss=0.02 if d.experts else 0.0)
            assert loss_gpu == loss_cpu and norm_gpu == norm_cpu, (step, loss_gpu, loss_cpu)
            for name in t.names:
                shape = d.tensor_shapes()[name]
                assert t.get(name, shape, t.GRAD).tobytes() == grads[name].tobytes(), (step, name)
                assert t.get(name, shape, t.M).tobytes() == m[name].tobytes(), (step, name)
                assert t.get(name, shape, t.V).tobytes() == v[name].tobytes(), (step, name)
        for name in t.names:
            assert t.get(name, d.tensor_shapes()[name]).tobytes() == params[name].tobytes(), name
    else:
        adapters = O.init_adapters(d, lora, 5)
        for name in adapters:
            if name.endswith(".lora_b"):
                adapters[name] = O.gaussian(len(name) + 7, *adapters[name].shape, scale=0.02)
        t = Trainer(gd, 256, 4, 128, lora=lora_config(lora.rank, lora.alpha, lora.targets, lora.rslora))
        t.load(weights)
        t.load(adapters)
        params = {n: a.copy() for n, a in adapters.items()}
        m = {n: np.zeros_like(a) for n, a in params.items()}
        v = {n: np.zeros_like(a) for n, a in params.items()}
        for step in (1, 2):
            loss_gpu, norm_gpu = t.step(windows, 1e-3, step)
            out: dict = {}
            loss_cpu, norm_cpu = O.lora_train_step(O.oracle_kernels(), od, weights, params, m, v, windows, opt, step,
                                                   2, lora, out=out)
            assert loss_gpu == loss_cpu and norm_gpu == norm_cpu, (step, loss_gpu, loss_cpu)
            for name, a in params.items():
                assert t.get(name, a.shape).tobytes() == a.tobytes(), (step, name)
                assert t.get(name, a.shape, t.M).tobytes() == m[name].tobytes(), (step, name)
                assert t.get(name, a.shape, t.V).tobytes() == v[name].tobytes(), (step, name)
            for name in O.lora_target_weights(d, lora):
                shape = d.tensor_shapes()[name]
                assert t.get(name, shape, t.GRAD).tobytes() == out["weight_grads"][name].tobytes(), (step, name)
    t.close()


NORM_CASES = {
    # OLMo 2: RMSNorm on each block's output before the residual add, whole-projection QK-norm, untied head
    "post": O.Decoder("olmo2", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=2, head_dim=16, eps=1e-6,
                      rope_theta=5e5, tied=False, qk_norm=2, norm_placement=1),
    # both placements (the Gemma layout's norms) with a residual multiplier folded into the output projections
    "sandwich": O.Decoder("llama", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=2, head_dim=16,
                          eps=1e-5, rope_theta=1e4, tied=True, norm_placement=2, residual_multiplier=0.5),
    # Gemma 3's layout at a larger shape, with Gemma 2's soft-capped scores and logits: unit-offset norms, GELU-tanh,
    # the window on layer 0 only (rotating with its own base), per-head QK-norm
    "gemma": O.Decoder("gemma3", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=2, head_dim=16, eps=1e-6,
                       rope_theta=1e6, tied=True, qk_norm=1, norm_placement=2, unit_offset=True, activation=1,
                       window=9, window_layers=(0,), local_rope_theta=1e4, embedding_multiplier=8.0,
                       attention_multiplier=0.25, attention_softcap=0.8, logits_softcap=2.0),
    # Gemma's real head size (256) with one kv head, and Phi-3-mini's (96)
    "head256": O.Decoder("gemma2", vocab=256, hidden=64, inter=96, layers=2, heads=2, kv_heads=1, head_dim=256,
                         eps=1e-6, rope_theta=1e4, tied=True, norm_placement=2, unit_offset=True, activation=1,
                         window=20, window_layers=(0,), embedding_multiplier=8.0, attention_multiplier=0.0625,
                         attention_softcap=50.0, logits_softcap=30.0),
    "head96": O.Decoder("phi3", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=4, head_dim=96,
                        eps=1e-5, rope_theta=1e4, tied=False, window=40),
    # post norms around routed experts (backprop.py:224-229, 462-463: the experts' sum is the normalised MLP output)
    "post_moe": O.Decoder("olmoe", vocab=256, hidden=64, inter=48, layers=2, heads=4, kv_heads=2, head_dim=16,
                          eps=1e-6, rope_theta=5e5, tied=False, qk_norm=2, norm_placement=1, experts=4, topk=2,
                          normalize=False),
    # sandwich norms with unit offsets around routed experts and a gated shared expert, layer 0 dense
    "sandwich_moe": O.Decoder("qwen2_moe", vocab=256, hidden=64, inter=96, layers=2, heads=4, kv_heads=2,
                              head_dim=16, eps=1e-5, rope_theta=1e4, tied=True, norm_placement=2, unit_offset=True,
                              experts=4, topk=2, normalize=True, expert_inter=24, shared_inter=40, shared_gate=True,
                              dense_layers=(0,)),
}


@pytest.mark.parametrize("case", sorted(NORM_CASES))
def test_norm_placement_step_matches_the_oracle(case):
    """Post and sandwich norm placement (backprop.py:222-287, 452-463): two steps over ragged windows, every gradient,
    parameter and moment against the oracle."""
    d = NORM_CASES[case]
    weights = O.synthetic_weights(d, seed=41, scale=0.05)
    rng = O.Random(43)
    windows = [[rng.next_u64() % d.vocab for _ in range(n)] for n in (33, 2, 70, 17)]
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
