"""GPU parity at the benchmark configurations' real layer shapes (tests/realshape.py): the device-resident step
against the oracle's step over the reference's own kernels, every gradient, parameter and AdamW moment after every
step compared bit for bit (through the SHA-256 digests tests/golden/make_realshape_goldens.py recorded from the
oracle), plus the loss and the gradient norm as exact doubles.

These reach the code paths the step selects by size at the bench's shapes and that the small fixtures never select:
the windows-in-sequence tied-embedding dW (>= 2048 output tiles), the vectorised weight transposes, the 4-way window
sums, cross-entropy at vocab 151936, the attention tiles at T = 2048, LoRA over a Q8_0 base at Qwen3-0.6B shapes, and
64-expert top-8 routing with the load-balancing loss at OLMoE shapes."""

from __future__ import annotations

import json
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

import oracle_lib as O
import realshape as R

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).parent / "golden"


def recorded(name: str) -> dict:
    path = GOLDEN / f"realshape_{name}.json"
    if not path.exists():
        pytest.skip(f"{path.name} not generated")
    return json.loads(path.read_text())


def make_trainer(cfg: R.RealShape):
    from etalii_dllm_amd.trainer import Decoder, Trainer, lora_config

    d = cfg.decoder
    decoder = Decoder(d.vocab, d.hidden, d.inter, d.layers, d.heads, d.kv_heads, d.head_dim, d.eps, d.rope_theta,
                      d.tied, d.attn_bias, d.qk_norm, d.window, d.experts, d.topk, d.normalize, d.expert_inter,
                      rotary_dim=d.rotary_dim, rope_scaling=d.scaling(), embedding_multiplier=d.embedding_multiplier,
                      attention_multiplier=d.attention_multiplier, residual_multiplier=d.residual_multiplier,
                      logits_scaling=d.logits_scaling, dense_layers=d.dense_layers, norm_placement=d.norm_placement,
                      norm_unit_offset=d.unit_offset, activation=d.activation, window_layers=d.window_layers,
                      local_rope_theta=d.local_rope_theta, attention_softcap=d.attention_softcap,
                      logits_softcap=d.logits_softcap, shared_inter=d.shared_inter, shared_gate=d.shared_gate)
    lora = None
    if cfg.lora is not None:
        lora = lora_config(cfg.lora.rank, cfg.lora.alpha, cfg.lora.targets, cfg.lora.rslora, cfg.base_quantize)
    tokens = sum(n - 1 for n in cfg.windows)
    return Trainer(decoder, tokens, len(cfg.windows), max(cfg.windows) - 1, lora=lora)


def compare(t, shapes: dict, step_record: dict, loss: float, norm: float) -> list[str]:
    bad = []
    if R.double_hex(loss) != step_record["loss"]:
        bad.append(f"loss {loss!r} != {float.fromhex(step_record['loss'])!r}")
    if R.double_hex(norm) != step_record["norm"]:
        bad.append(f"norm {norm!r} != {float.fromhex(step_record['norm'])!r}")
    which = {"param": t.PARAM, "grad": t.GRAD, "m": t.M, "v": t.V}
    jobs = [(name, kind, want) for name, digests in step_record["tensors"].items() for kind, want in digests.items()]

    def check(job):
        name, kind, want = job
        return None if R.digest(t.get(name, shapes[name], which[kind])) == want else f"{name} {kind}"

    # the copies and the hashing of many tensors (the 6.92 B-parameter arena at full depth) on a thread pool
    with ThreadPoolExecutor(max_workers=R.WORKERS) as pool:
        bad += [b for b in pool.map(check, jobs) if b is not None]
    return bad


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", sorted(R.CONFIGS))
def test_step_at_real_shape_matches_the_oracle(name):
    record = recorded(name)
    cfg = R.CONFIGS[name]
    d = cfg.decoder
    base = R.weights(cfg)
    assert R.digest_of_concatenation(base.values()) == record["inputs"], "the input generator differs from the recording's"
    t = make_trainer(cfg)
    try:
        t.load(base)
        shapes = dict(d.tensor_shapes())
        if cfg.lora is not None:
            adapters = R.adapters(cfg)
            assert R.digest(O.concatenated(adapters)) == record["adapter_inputs"]
            t.load(adapters)
            shapes.update(O.adapter_shapes(d, cfg.lora))
        del base
        windows = R.windows(cfg)
        for step, step_record in enumerate(record["steps"], start=1):
            loss, norm = t.step(windows, cfg.learning_rate, step, router_aux_loss=cfg.router_aux_loss)
            bad = compare(t, shapes, step_record, loss, norm)
            print(f"{name} step {step}: loss {loss!r} norm {norm!r}, {len(bad)} mismatches", flush=True)
            if bad:
                print("mismatches:", " | ".join(bad), flush=True)
            assert not bad, f"{name} step {step}: {len(bad)} mismatches, first {bad[:12]}"
    finally:
        t.close()

