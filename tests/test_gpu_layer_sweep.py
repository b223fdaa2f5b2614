"""GPU parity at the per-op microbench configuration: Qwen2.5-0.5B layer shapes (hidden 896, 14 query / 2 KV heads of
64, SwiGLU intermediate 4864, RoPE theta 1e6), weights N(0, 0.02), activations N(0, 1), upstream gradients
N(0, 1e-3), with the row count M swept over {1, 7, 64, 2048, 8192}.

Row-local outputs (linear, dX, RMSNorm forward and dx, RoPE, SiLU/SwiGLU and their gradients, attention out and dq)
must be bit-identical for every M: each M's rows equal the first M rows of the largest run. Reductions over rows (dW,
db, the norm weight's dw, dk, dv) must equal the CPU oracle at each M: dW and db on a subset of their outputs (each
output's chain runs over the rows only, so the oracle on the matching columns of x and dy gives those outputs
exactly), the norm's dw whole, dk and dv whole where the oracle's attention finishes in seconds (M <= 64) and, at every
M, on the last keys: only the last queries see them, so the oracle's attention backward of those queries over all M
keys (a cached-prefix call) gives their dk and dv exactly. AdamW runs once over the layer's 14.9 M parameters.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

HIDDEN, INTER, HEADS, KV_HEADS, HEAD_DIM, THETA = 896, 4864, 14, 2, 64, 1e6
SWEEP = (1, 7, 64, 2048, 8192)
M_MAX = SWEEP[-1]
ATTN_TAIL = 16  # last keys (and queries) checked against the oracle at every M
COLS_OUT = np.array([0, 1, 63, 64, 127, 300, 895])  # sampled output features (< 896) for dW / db
COLS_IN = np.array([0, 5, 127, 128, 511, 890, 895])  # sampled input features (< 896)


@pytest.fixture(scope="module")
def K():
    from etalii_dllm_amd import kernels

    return kernels


@pytest.fixture(scope="module")
def ora():
    return O.oracle_kernels()


@pytest.fixture(scope="module")
def data():
    d = {
        "wq": O.gaussian(101, HIDDEN, HIDDEN, scale=0.02),
        "wk": O.gaussian(102, KV_HEADS * HEAD_DIM, HIDDEN, scale=0.02),
        "wgate": O.gaussian(103, INTER, HIDDEN, scale=0.02),
        "wdown": O.gaussian(104, HIDDEN, INTER, scale=0.02),
        "wnorm": O.gaussian(105, HIDDEN, scale=0.02) + np.float32(1.0),
        "x": O.gaussian(111, M_MAX, HIDDEN),
        "xi": O.gaussian(112, M_MAX, INTER),
        "dyh": O.gaussian(121, M_MAX, HIDDEN, scale=1e-3),
        "dyk": O.gaussian(122, M_MAX, KV_HEADS * HEAD_DIM, scale=1e-3),
        "dyi": O.gaussian(123, M_MAX, INTER, scale=1e-3),
    }
    return d


def assert_same(a, b, what=""):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.tobytes() != b.tobytes():
        diff = np.flatnonzero(a.view(np.uint32).ravel() != b.view(np.uint32).ravel())
        raise AssertionError(f"{what}: {len(diff)} of {a.size} elements differ, first at {diff[:5]}")


LINEARS = [  # (name, x key, weight key, dy key)
    ("q", "x", "wq", "dyh"),
    ("k", "x", "wk", "dyk"),
    ("gate", "x", "wgate", "dyi"),
    ("down", "xi", "wdown", "dyh"),
]


@pytest.mark.parametrize(("name", "xk", "wk", "dyk"), LINEARS)
def test_linear_sweep_rows_invariant_and_weight_gradients_match_the_oracle(K, ora, data, name, xk, wk, dyk):
    x, w, dy = data[xk], data[wk], data[dyk]
    full_out = K.linear(x, w)
    full_dx, _, _ = K.linear_backward(x, w, dy, True)
    n_out = w.shape[0]
    outs = COLS_OUT[COLS_OUT < n_out]
    ins = COLS_IN[COLS_IN < w.shape[1]] if w.shape[1] == HIDDEN else np.array([0, 7, 1000, 4095, 4863])
    for m in SWEEP:
        assert_same(K.linear(x[:m], w), full_out[:m], f"{name} forward M={m}")
        dx, dw, db = K.linear_backward(x[:m], w, dy[:m], True)
        assert_same(dx, full_dx[:m], f"{name} dX M={m}")
        xs = np.ascontiguousarray(x[:m][:, ins])
        dys = np.ascontiguousarray(dy[:m][:, outs])
        _, want_dw, want_db = ora.linear_backward(xs, np.ascontiguousarray(w[outs][:, ins]), dys, True)
        assert_same(dw[np.ix_(outs, ins)], want_dw, f"{name} dW M={m}")
        assert_same(db[outs], want_db, f"{name} db M={m}")


def test_rms_norm_sweep(K, ora, data):
    x, w, dy = data["x"], data["wnorm"], data["dyh"]
    full = K.rms_norm(x, w, 1e-6)
    full_dx, _ = K.rms_norm_backward(x, w, dy, 1e-6)
    for m in SWEEP:
        assert_same(K.rms_norm(x[:m], w, 1e-6), full[:m], f"rms_norm M={m}")
        dx, dw = K.rms_norm_backward(x[:m], w, dy[:m], 1e-6)
        assert_same(dx, full_dx[:m], f"rms_norm dx M={m}")
        _, want_dw = ora.rms_norm_backward(x[:m], w, dy[:m], 1e-6)
        assert_same(dw, want_dw, f"rms_norm dw M={m}")


def test_rope_sweep(K, ora, data):
    q = data["x"][:, : HEADS * HEAD_DIM].reshape(M_MAX, HEADS, HEAD_DIM)
    pos = np.arange(M_MAX, dtype=np.int64)
    inv = O.rope_inv_freq(HEAD_DIM, THETA)
    for inverse in (False, True):
        full = K.rope(q, pos, inv, False, inverse)
        assert_same(full, ora.rope(q, pos, inv, False, inverse), f"rope inverse={inverse} M={M_MAX}")
        for m in SWEEP[:-1]:
            assert_same(K.rope(q[:m], pos[:m], inv, False, inverse), full[:m], f"rope inverse={inverse} M={m}")


def test_swiglu_sweep(K, ora, data):
    gate, up, dy = data["xi"], data["dyi"] * np.float32(1000.0), data["dyi"]
    full_act, full_prod, full_dsilu = K.silu(gate), K.swiglu(gate, up), K.silu_backward(gate, dy)
    for m in SWEEP:
        assert_same(K.silu(gate[:m]), full_act[:m], f"silu M={m}")
        assert_same(K.swiglu(gate[:m], up[:m]), full_prod[:m], f"swiglu M={m}")
        assert_same(K.silu_backward(gate[:m], dy[:m]), full_dsilu[:m], f"silu_backward M={m}")
    m = 64
    assert_same(full_act[:m], ora.silu(gate[:m]), "silu vs oracle")
    assert_same(full_prod[:m], ora.swiglu(gate[:m], up[:m]), "swiglu vs oracle")
    assert_same(full_dsilu[:m], ora.silu_backward(gate[:m], dy[:m]), "silu_backward vs oracle")


def test_causal_gqa_attention_sweep(K, ora, data):
    n = M_MAX
    q = data["x"][:n, : HEADS * HEAD_DIM].reshape(n, HEADS, HEAD_DIM)
    k = O.gaussian(131, n, KV_HEADS, HEAD_DIM)
    v = O.gaussian(132, n, KV_HEADS, HEAD_DIM)
    dout = O.gaussian(133, n, HEADS, HEAD_DIM, scale=1e-3)
    scale = 1.0 / np.sqrt(HEAD_DIM)
    full_out = K.attention(q, k, v, scale, True)
    full_dq, _, _ = K.attention_backward(q, k, v, dout, scale, True)
    for m in SWEEP:
        args = (q[:m], k[:m], v[:m])
        out = K.attention(*args, scale, True)
        dq, dk, dv = K.attention_backward(*args, dout[:m], scale, True)
        assert_same(out, full_out[:m], f"attention out M={m}")
        assert_same(dq, full_dq[:m], f"attention dq M={m}")
        s = min(m, ATTN_TAIL)
        tail = (q[m - s:m], k[:m], v[:m])
        want_out = ora.attention(*tail, scale, True, m - s)
        want = ora.attention_backward(*tail, dout[m - s:m], scale, True, m - s)
        assert_same(out[m - s:], want_out, f"attention out of the last queries vs oracle M={m}")
        assert_same(dq[m - s:], want[0], f"attention dq of the last queries vs oracle M={m}")
        assert_same(dk[m - s:], want[1][m - s:], f"attention dk of the last keys vs oracle M={m}")
        assert_same(dv[m - s:], want[2][m - s:], f"attention dv of the last keys vs oracle M={m}")
        # the same tail through the row kernels (a cached-prefix call), past 2048 keys where M is
        got_tail = K.attention_backward(*tail, dout[m - s:m], scale, True, m - s)
        for g, w, what in zip(got_tail, want, ("dq", "dk", "dv")):
            assert_same(g, w, f"cached-prefix attention {what} M={m}")
        if m <= 64:
            assert_same(out, ora.attention(*args, scale, True), f"attention out vs oracle M={m}")
            want = ora.attention_backward(*args, dout[:m], scale, True)
            for got, exp, what in zip((dq, dk, dv), want, ("dq", "dk", "dv")):
                assert_same(got, exp, f"attention {what} vs oracle M={m}")


def test_adamw_over_the_layer_parameters(K, ora, data):
    """One fused AdamW update over the layer's q, k, v, o, gate, up and down weights and its two norm weights."""
    n = 2 * HIDDEN * HIDDEN + 2 * KV_HEADS * HEAD_DIM * HIDDEN + 3 * INTER * HIDDEN + 2 * HIDDEN
    param = O.gaussian(141, n, scale=0.02)
    grad = O.gaussian(142, n, scale=1e-3)
    m1 = O.gaussian(143, n, scale=1e-4)
    m2 = np.abs(O.gaussian(144, n, scale=1e-6))
    args = (1e-4, 0.9, 0.999, 1e-8, 0.01, 1.0 - 0.9 ** 3, 1.0 - 0.999 ** 3, 0.5)
    gp, gm, gv = param.copy(), m1.copy(), m2.copy()
    K.adamw_step(gp, grad, gm, gv, *args)
    op, om, ov = param.copy(), m1.copy(), m2.copy()
    ora.adamw_step(op, grad, om, ov, *args)
    assert_same(gp, op, "param")
    assert_same(gm, om, "m")
    assert_same(gv, ov, "v")
