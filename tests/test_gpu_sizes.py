"""GPU parity of the step at sizes outside the matrix-core kernel's comfort zone, against the oracle's step.

The reference takes any model size, any token count and any depth (architecture.py:175-254 checks only the head
counts and the layer indices; trainer.py:312-335 loops over windows with no cap). These steps check that the trainer
does too, bit for bit:
- sizes that are not whole 16-byte chunks (vocabulary 301, intermediate 30, 6 experts of 18), whose matmuls widen
  their A operand into a double scratch and run on the VALU kernels, and whose weight transposes take the scalar
  branch of the batched transpose;
- a step of 67,584 tokens in 66 windows (past 65,535 rows and past the 64 windows one column-sum launch takes);
- a 66-layer model with per-layer dense and windowed choices past layer 63.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O
from test_gpu_trainer import make_trainer

pytestmark = pytest.mark.gpu


def check_steps(d: O.Decoder, windows, steps=2, router_aux_loss=0.0, seed=11, max_window=None):
    weights = O.synthetic_weights(d, seed=seed, scale=0.05)
    total = sum(len(w) - 1 for w in windows)
    longest = max(len(w) - 1 for w in windows)
    t = make_trainer(d, weights, max_tokens=total, max_windows=len(windows), max_window=max_window or longest)
    params = {n: a.copy() for n, a in weights.items()}
    m = {n: np.zeros_like(a) for n, a in params.items()}
    v = {n: np.zeros_like(a) for n, a in params.items()}
    opt = O.AdamWConfig(learning_rate=1e-3, schedule="constant")
    for step in range(1, steps + 1):
        print(f"[sizes] {d.family} step {step}: {len(windows)} windows, {total} rows", flush=True)
        loss_gpu, norm_gpu = t.step(windows, 1e-3, step, router_aux_loss=router_aux_loss)
        loss_cpu, _, norm_cpu, grads = O.train_step(O.oracle_kernels(), d, params, m, v, windows, opt, step, steps,
                                                    router_aux_loss=router_aux_loss)
        assert loss_gpu == loss_cpu and norm_gpu == norm_cpu
        for name in t.names:
            shape = d.tensor_shapes()[name]
            assert t.get(name, shape, t.GRAD).tobytes() == grads[name].tobytes(), name
            assert t.get(name, shape).tobytes() == params[name].tobytes(), name
            assert t.get(name, shape, t.M).tobytes() == m[name].tobytes(), name
            assert t.get(name, shape, t.V).tobytes() == v[name].tobytes(), name
    t.close()


def ragged_windows(vocab, lengths, seed):
    rng = O.Random(seed)
    return [[rng.next_u64() % vocab for _ in range(n)] for n in lengths]


@pytest.mark.parametrize("tied", [True, False])
def test_sizes_that_are_not_whole_chunks(tied):
    """Vocabulary 301, hidden 36, intermediate 30, q/k/v biases: every matmul touching the vocabulary or the
    intermediate size runs on the widened VALU path, the rest on the matrix cores; two steps over ragged windows."""
    d = O.Decoder("qwen2", vocab=301, hidden=36, inter=30, layers=2, heads=3, kv_heads=1, head_dim=12, eps=1e-6,
                  rope_theta=1e6, tied=tied, attn_bias=True)
    check_steps(d, ragged_windows(d.vocab, (33, 2, 70, 17), 5))


def test_expert_sizes_that_are_not_whole_chunks():
    """6 experts of 18 (top 2) and vocabulary 301: the router and every expert matmul run one launch each on the
    widened path; two steps with the load-balancing loss."""
    d = O.Decoder("olmoe", vocab=301, hidden=36, inter=30, layers=2, heads=3, kv_heads=3, head_dim=12, eps=1e-5,
                  rope_theta=1e4, tied=False, qk_norm=2, experts=6, topk=2, normalize=False, expert_inter=18)
    check_steps(d, ragged_windows(d.vocab, (33, 2, 70, 17), 6), router_aux_loss=0.05)


def test_step_of_more_than_65535_tokens():
    """66 windows of 1024 targets (67,584 rows in one step): the packed rows past 65,535 and more windows than one
    column-sum launch takes (64), one step against the oracle."""
    d = O.Decoder("llama", vocab=64, hidden=32, inter=32, layers=1, heads=2, kv_heads=1, head_dim=16, eps=1e-5,
                  rope_theta=1e4, tied=True)
    check_steps(d, ragged_windows(d.vocab, [1025] * 66, 7), steps=1)


def test_per_layer_choices_past_layer_64():
    """66 layers with routed experts, layers 1 and 65 dense, and a sliding window on layers 0, 64 and 65 only:
    per-layer choices past the 64 a bit mask holds, two steps against the oracle."""
    d = O.Decoder("qwen3_moe", vocab=64, hidden=16, inter=24, layers=66, heads=2, kv_heads=1, head_dim=8, eps=1e-6,
                  rope_theta=1e6, tied=True, qk_norm=1, window=5, window_layers=(0, 64, 65), experts=4, topk=2,
                  normalize=True, expert_inter=8, dense_layers=(1, 65))
    check_steps(d, ragged_windows(d.vocab, (20, 9), 8), router_aux_loss=0.01)
