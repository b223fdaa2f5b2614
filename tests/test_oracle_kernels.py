"""Per-kernel pins of the oracle: bit equality with the reference's own kernels (oracle/_ref, built from the reference
headers; skipped where that prebuilt library is absent), and closed forms / invariants that a dropped term, a wrong
sign or a transposed operand would break (the reference's float64 yardsticks, tests/test_training.py:78-229)."""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle_lib as O

needs_ref = pytest.mark.skipif(not O.reference_available(), reason="oracle/_ref not built (no reference checkout)")


def adversarial(seed: int, *shape: int) -> np.ndarray:
    """Values spanning 1e-30 .. 1e20 with both signs and exact zeros (reference test_batch_invariance.py:68-78)."""
    values = O.gaussian(seed, *shape).astype(np.float64)
    exponents = O.gaussian(seed + 1000, *shape).astype(np.float64)
    out = values * np.power(10.0, np.clip(np.round(exponents * 8), -30, 20))
    out[np.abs(O.gaussian(seed + 2000, *shape)) < 0.05] = 0.0
    return out.astype(np.float32)


def same(a, b) -> bool:
    return np.asarray(a).tobytes() == np.asarray(b).tobytes()


@needs_ref
def test_math_matches_reference():
    o, r = O.oracle(), O.ref()
    xs = np.concatenate([O.gaussian(1, 4000).astype(np.float64) * 30, np.linspace(-800, 800, 3001),
                         [0.0, -0.0, 1e-300, 5e-324, 709.7, 709.79, -745.1, -745.3, 1e6, 3e7, np.inf, -np.inf]])
    for name in ("exp", "log", "sin", "cos", "tanh", "sigmoid"):
        for x in xs:
            a, b = getattr(o, "orc_" + name)(float(x)), getattr(r, "ref_" + name)(float(x))
            assert (math.isnan(a) and math.isnan(b)) or np.float64(a).tobytes() == np.float64(b).tobytes(), (name, x)


@needs_ref
@pytest.mark.parametrize("rows", [1, 7, 33])
def test_linear_and_backward_match_reference(rows):
    o, r = O.oracle_kernels(), O.ref_kernels()
    x, w, b, dy = adversarial(1, rows, 37), adversarial(2, 19, 37), adversarial(3, 19), adversarial(4, rows, 19)
    assert same(o.linear(x, w, b), r.linear(x, w, b))
    for a, c in zip(o.linear_backward(x, w, dy, True), r.linear_backward(x, w, dy, True)):
        assert same(a, c)


@needs_ref
def test_row_kernels_match_reference():
    o, r = O.oracle_kernels(), O.ref_kernels()
    x, w, dy = O.gaussian(5, 9, 48, scale=3.0), O.gaussian(6, 48), O.gaussian(7, 9, 48)
    assert same(o.rms_norm(x, w, 1e-5), r.rms_norm(x, w, 1e-5))
    assert same(o.rms_norm(x, w, 1e-6, True), r.rms_norm(x, w, 1e-6, True))
    for a, c in zip(o.rms_norm_backward(x, w, dy, 1e-5), r.rms_norm_backward(x, w, dy, 1e-5)):
        assert same(a, c)
    g, up = O.gaussian(8, 500, scale=6.0), O.gaussian(11, 500)
    assert same(o.silu(g), r.silu(g))
    assert same(o.swiglu(g, up), r.swiglu(g, up))
    assert same(o.silu_backward(g, up), r.silu_backward(g, up))
    q = O.gaussian(9, 11, 3, 16)
    pos = np.arange(11, dtype=np.int64) * 131
    for inv in (O.rope_inv_freq(16, 1e6), O.rope_inv_freq(8, 1e4)):
        for interleaved in (False, True):
            for inverse in (False, True):
                assert same(o.rope(q, pos, inv, interleaved, inverse), r.rope(q, pos, inv, interleaved, inverse))


@needs_ref
@pytest.mark.parametrize(("q_len", "kv_len", "window", "softcap", "offset"),
                         [(9, 9, 0, 0.0, 0), (5, 9, 0, 0.0, 4), (9, 9, 3, 0.0, 0), (9, 9, 0, 0.7, 0)])
def test_attention_matches_reference(q_len, kv_len, window, softcap, offset):
    o, r = O.oracle_kernels(), O.ref_kernels()
    q, k, v = O.gaussian(12, q_len, 6, 8), O.gaussian(13, kv_len, 2, 8), O.gaussian(14, kv_len, 2, 8)
    dout = O.gaussian(15, q_len, 6, 8)
    args = (0.35, True, offset, window, softcap)
    assert same(o.attention(q, k, v, *args), r.attention(q, k, v, *args))
    for a, c in zip(o.attention_backward(q, k, v, dout, *args), r.attention_backward(q, k, v, dout, *args)):
        assert same(a, c)


@needs_ref
def test_loss_embedding_optimizer_and_routing_match_reference():
    o, r = O.oracle_kernels(), O.ref_kernels()
    logits = O.gaussian(16, 6, 301, scale=4.0)
    targets = np.array([3, -1, 300, 0, 17, 17], np.int64)
    (la, da), (lb, db) = o.cross_entropy(logits, targets, 0.25), r.cross_entropy(logits, targets, 0.25)
    assert la == lb and same(da, db)
    dy, tokens = O.gaussian(17, 12, 5), np.array([3, 1, 3, 0, 3, 1, 9, 9, 9, 2, 0, 3], np.int64)
    assert same(o.embedding_backward(dy, tokens, 10), r.embedding_backward(dy, tokens, 10))
    g = adversarial(18, 1000)
    assert o.sum_squares(g) == r.sum_squares(g)
    p, grad = O.gaussian(18, 300), O.gaussian(19, 300)
    m, v = O.gaussian(20, 300, scale=0.1), np.abs(O.gaussian(21, 300, scale=0.1))
    pa, ma, va = p.copy(), m.copy(), v.copy()
    pb, mb, vb = p.copy(), m.copy(), v.copy()
    o.adamw_step(pa, grad, ma, va, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1 - 0.9**3, 1 - 0.999**3, 0.5)
    r.adamw_step(pb, grad, mb, vb, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1 - 0.9**3, 1 - 0.999**3, 0.5)
    assert same(pa, pb) and same(ma, mb) and same(va, vb)
    rl = O.gaussian(22, 20, 8, scale=3.0)
    for normalize in (False, True):
        ia, wa = o.moe_route(rl, 3, normalize)
        ib, wb = r.moe_route(rl, 3, normalize)
        assert same(ia, ib) and same(wa, wb)
        dw, dp = O.gaussian(23, 20, 3), O.gaussian(24, 20, 8)
        assert same(o.moe_route_backward(rl, ia, dw, dp, normalize), r.moe_route_backward(rl, ia, dw, dp, normalize))
        assert same(o.moe_route_backward(rl, ia, dw, None, normalize),
                    r.moe_route_backward(rl, ia, dw, None, normalize))
    assert same(o.column_mean(rl), r.column_mean(rl))
    assert same(o.softmax(rl[0].copy()), r.softmax(rl[0].copy()))


# ---- closed forms and invariants (no reference needed) ----

def close(ours, reference, tolerance=1e-5):
    reference = np.asarray(reference, dtype=np.float64)
    scale = max(1.0, float(np.abs(reference).max()))
    np.testing.assert_allclose(np.asarray(ours, np.float64), reference, rtol=0, atol=tolerance * scale)


def test_math_special_values_and_accuracy():
    o = O.oracle()
    assert o.orc_exp(0.0) == 1.0 and o.orc_log(1.0) == 0.0 and o.orc_sin(0.0) == 0.0 and o.orc_cos(0.0) == 1.0
    assert o.orc_exp(-800.0) == 0.0 and o.orc_exp(800.0) == math.inf and math.isnan(o.orc_log(-1.0))
    xs = np.linspace(-50, 50, 2001)
    assert max(abs(o.orc_exp(x) / math.exp(x) - 1) for x in xs) < 1e-14
    assert max(abs(o.orc_log(math.exp(x)) - x) for x in xs) < 1e-13
    assert max(abs(o.orc_sin(x) - math.sin(x)) for x in xs) < 1e-14
    assert max(abs(o.orc_cos(x) - math.cos(x)) for x in xs) < 1e-14
    assert max(abs(o.orc_tanh(x) - math.tanh(x)) for x in xs) < 1e-15
    assert all(o.orc_tanh(-x) == -o.orc_tanh(x) for x in xs)


def test_linear_backward_matches_float64():
    k = O.oracle_kernels()
    x, w, dy = O.gaussian(1, 5, 7), O.gaussian(2, 3, 7), O.gaussian(4, 5, 3)
    dx, dw, db = k.linear_backward(x, w, dy, True)
    x64, w64, dy64 = (a.astype(np.float64) for a in (x, w, dy))
    close(dx, dy64 @ w64)
    close(dw, dy64.T @ x64)
    close(db, dy64.sum(0))
    assert same(k.linear_backward(x[2:3].copy(), w, dy[2:3].copy())[0], dx[2:3])


def numeric_gradient(f, x, eps=1e-6):
    grad = np.zeros_like(x, dtype=np.float64)
    for index in np.ndindex(x.shape):
        plus, minus = x.astype(np.float64), x.astype(np.float64)
        plus[index] += eps
        minus[index] -= eps
        grad[index] = (f(plus) - f(minus)) / (2 * eps)
    return grad


def test_rms_norm_backward_matches_numeric_gradient():
    k = O.oracle_kernels()
    x, w, dy = O.gaussian(5, 3, 8), O.gaussian(6, 8), O.gaussian(7, 3, 8)
    eps = 1e-5
    dx, dw = k.rms_norm_backward(x, w, dy, eps)

    def forward(xv, wv):
        return xv / np.sqrt(np.mean(xv * xv, -1, keepdims=True) + eps) * wv

    close(dx, numeric_gradient(lambda a: float((forward(a, w) * dy).sum()), x), 1e-6)
    close(dw, numeric_gradient(lambda a: float((forward(x.astype(np.float64), a) * dy).sum()), w), 1e-6)


def test_silu_backward_matches_numeric_gradient():
    k = O.oracle_kernels()
    x, dy = O.gaussian(8, 20, scale=4.0), O.gaussian(9, 20)
    reference = numeric_gradient(lambda a: float((a / (1 + np.exp(-a)) * dy).sum()), x)
    close(k.silu_backward(x, dy), reference, 1e-7)


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_inverse_is_the_transpose(interleaved):
    k = O.oracle_kernels()
    x, dy = O.gaussian(10, 5, 2, 8), O.gaussian(11, 5, 2, 8)
    positions, inv = np.arange(3, 8, dtype=np.int64), O.rope_inv_freq(8, 10000.0)
    rotated = k.rope(x, positions, inv, interleaved).astype(np.float64)
    back = k.rope(dy, positions, inv, interleaved, True).astype(np.float64)
    assert abs((rotated * dy).sum() - (x.astype(np.float64) * back).sum()) < 1e-5
    close(k.rope(rotated.astype(np.float32), positions, inv, interleaved, True), x, 1e-6)


def reference_attention(q, k, v, scale, window=None):
    q_len, heads, _ = q.shape
    group = heads // k.shape[1]
    out = np.zeros((q_len, heads, v.shape[2]))
    offset = k.shape[0] - q_len
    for h in range(heads):
        scores = q[:, h] @ k[:, h // group].T * scale
        scores = scores + np.triu(np.full(scores.shape, -np.inf), offset + 1)
        if window is not None:
            scores = scores + np.tril(np.full(scores.shape, -np.inf), offset - window)
        p = np.exp(scores - scores.max(-1, keepdims=True))
        out[:, h] = (p / p.sum(-1, keepdims=True)) @ v[:, h // group]
    return out


@pytest.mark.parametrize(("q_len", "window"), [(4, None), (2, None), (4, 2)])
def test_attention_backward_matches_numeric_gradient(q_len, window):
    kern = O.oracle_kernels()
    q, k, v = O.gaussian(12, q_len, 4, 6), O.gaussian(13, 4, 2, 6), O.gaussian(14, 4, 2, 6)
    dout = O.gaussian(15, q_len, 4, 6)
    scale = 1 / np.sqrt(6)
    dq, dk, dv = kern.attention_backward(q, k, v, dout, scale, True, 4 - q_len, window or 0)
    q64, k64, v64 = (a.astype(np.float64) for a in (q, k, v))

    def loss(a, b, c):
        return float((reference_attention(a, b, c, scale, window) * dout).sum())

    close(dq, numeric_gradient(lambda a: loss(a, k64, v64), q), 1e-6)
    close(dk, numeric_gradient(lambda a: loss(q64, a, v64), k), 1e-6)
    close(dv, numeric_gradient(lambda a: loss(q64, k64, a), v), 1e-6)
    close(kern.attention(q, k, v, scale, True, 4 - q_len, window or 0), reference_attention(q64, k64, v64, scale,
                                                                                           window), 1e-6)


def test_cross_entropy_matches_float64():
    k = O.oracle_kernels()
    logits = O.gaussian(16, 4, 11, scale=3.0)
    targets = np.array([3, -1, 10, 0], np.int64)
    loss, dlogits = k.cross_entropy(logits, targets, 0.25)
    l64 = logits.astype(np.float64)
    lse = np.log(np.exp(l64 - l64.max(1, keepdims=True)).sum(1)) + l64.max(1)
    kept = targets >= 0
    assert abs(loss - float((lse - l64[np.arange(4), targets])[kept].sum())) < 1e-12
    probs = np.exp(l64 - lse[:, None])
    probs[np.arange(4)[kept], targets[kept]] -= 1
    probs[~kept] = 0
    close(dlogits, probs * 0.25, 1e-7)


def test_embedding_backward_sums_rows_per_token():
    k = O.oracle_kernels()
    dy, tokens = O.gaussian(17, 6, 5), np.array([3, 1, 3, 0, 3, 1], np.int64)
    expected = np.zeros((4, 5))
    np.add.at(expected, tokens, dy.astype(np.float64))
    close(k.embedding_backward(dy, tokens, 4), expected, 1e-7)
    with pytest.raises(ValueError):
        k.embedding_backward(dy, np.array([4, 0, 0, 0, 0, 0], np.int64), 4)


def test_adamw_step_is_the_documented_formula():
    """Bitwise against the float64 closed form (reference tests/test_training.py:217-229)."""
    k = O.oracle_kernels()
    param, grad = O.gaussian(18, 50), O.gaussian(19, 50)
    m, v = O.gaussian(20, 50, scale=0.1), np.abs(O.gaussian(21, 50, scale=0.1))
    p64, g64, m64, v64 = (a.astype(np.float64) for a in (param, grad, m, v))
    lr, b1, b2, eps, wd, c1, c2, s = 1e-3, 0.9, 0.999, 1e-8, 0.01, 1 - 0.9**3, 1 - 0.999**3, 0.5
    g = g64 * s
    m_new = (b1 * m64 + (1 - b1) * g).astype(np.float32)
    v_new = (b2 * v64 + (1 - b2) * g * g).astype(np.float32)
    expected = (p64 * (1 - lr * wd) - lr * (m_new / c1) / (np.sqrt(v_new / c2) + eps)).astype(np.float32)
    param, m, v = param.copy(), m.copy(), v.copy()
    k.adamw_step(param, grad, m, v, lr, b1, b2, eps, wd, c1, c2, s)
    assert same(param, expected) and same(m, m_new) and same(v, v_new)


def test_sum_squares_is_the_serial_double_chain():
    g = O.gaussian(30, 5000, scale=3.0)
    acc = 0.0
    for value in g.astype(np.float64):
        acc += value * value
    assert O.oracle_kernels().sum_squares(g) == acc


@pytest.mark.parametrize("name", sorted(O.q8_0_cases()))
def test_quantize_q8_0_matches_reference(name):
    x = O.q8_0_cases()[name]
    qa, sa = O.quantize_q8_0(O.oracle().orc_quantize_q8_0, x)
    qb, sb = O.quantize_q8_0(O.ref().ref_quantize_q8_0, x)
    assert qa.tobytes() == qb.tobytes() and sa.tobytes() == sb.tobytes()


def test_q8_0_round_trips_values_on_its_grid():
    """Values k * d for |k| <= 127 with one |k| = 127 quantise to k exactly and dequantise to k * d (closed form)."""
    rng = np.random.default_rng(5)
    k = rng.integers(-127, 128, size=(8, 32)).astype(np.float32)
    k[:, 0] = 127.0
    d = np.float32(0.25)
    x = (k * d).ravel()
    q, s = O.quantize_q8_0(O.oracle().orc_quantize_q8_0, x)
    assert np.all(s == d) and np.array_equal(q.astype(np.float32), k.ravel())
    assert O.dequantize_q8_0(q, s).tobytes() == x.tobytes()


def test_gelu_tanh_and_softcap_backward_match_reference():
    """grad.hpp:183-197 against the compiled reference, on Gaussians, large magnitudes and special values."""
    if not O.reference_available():
        pytest.skip("oracle/_ref not built")
    r = O.ref()
    x = np.concatenate([O.gaussian(31, 400, scale=3.0), adversarial(32, 200),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 1e4, np.inf, -np.inf, np.nan], np.float32)])
    dy = O.gaussian(33, x.size)
    want = np.array([r.ref_gelu_tanh_backward(float(a), float(b)) for a, b in zip(x, dy)], np.float32)
    assert same(O.gelu_tanh_backward(x, dy), want)
    assert same(O.gelu_tanh(x), np.array([r.ref_gelu_tanh(float(a)) for a in x], np.float32))
    for cap in (30.0, 50.0, 0.5):
        want = np.array([r.ref_softcap_backward(float(a), float(b), cap) for a, b in zip(x, dy)], np.float32)
        assert same(O.softcap_backward(x, dy, cap), want)


def test_gelu_tanh_matches_the_closed_form():
    """nn.hpp:481-485 against numpy's tanh in double, rounded once: within one float ulp for x >= -4 (the portable tanh
    differs from libm's by a few double ulps, which moves a float rounding at most one step), and within 1e-13
    absolutely in the negative tail, where 1 + tanh cancels and those double ulps dominate the tiny result."""
    x = np.concatenate([O.gaussian(35, 2000, scale=3.0), np.array([0.0, -0.0, 30.0, -30.0, 1e-20], np.float32)])
    c = np.sqrt(2.0 / np.pi)
    d = x.astype(np.float64)
    want = (0.5 * d * (1.0 + np.tanh(c * (d + 0.044715 * d * d * d)))).astype(np.float32)
    got = O.gelu_tanh(x)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert np.all(ulps[x >= -4] <= 1)
    assert np.all(np.abs(got.astype(np.float64) - want.astype(np.float64)) <= 1e-13)
    assert got[-5] == 0.0 and got[-3] == np.float32(30.0) and got[-2] == 0.0


def test_gelu_tanh_and_softcap_backward_match_numeric_gradients():
    x = O.gaussian(34, 64, scale=2.0).astype(np.float64)
    h = 1e-4
    c = np.sqrt(2.0 / np.pi)
    gelu = lambda v: 0.5 * v * (1.0 + np.tanh(c * (v + 0.044715 * v ** 3)))  # noqa: E731
    close(O.gelu_tanh_backward(x.astype(np.float32), np.ones(64, np.float32)),
          (gelu(x.astype(np.float32).astype(np.float64) + h) - gelu(x.astype(np.float32).astype(np.float64) - h)) / (2 * h), 1e-6)
    cap = 5.0
    soft = lambda v: cap * np.tanh(v / cap)  # noqa: E731
    xf = x.astype(np.float32).astype(np.float64)
    close(O.softcap_backward(x.astype(np.float32), np.ones(64, np.float32), cap), (soft(xf + h) - soft(xf - h)) / (2 * h), 1e-6)


def q8_linear_case(seed: int, rows: int, in_f: int, out_f: int):
    x = O.gaussian(seed, rows, in_f)
    x[0, :32] = 0.0  # an all-zero block: scale 0
    if rows > 2:
        x[2, 5] = np.inf  # a non-finite value is quantised as 0 and left out of the block's amax
        x[2, 40 % in_f] = -7e30
    w = O.gaussian(seed + 1, out_f, in_f, scale=0.02)
    q, s = O.quantize_q8_0(O.oracle().orc_quantize_q8_0, w)
    return x, q.reshape(out_f, in_f), s.reshape(out_f, in_f // 32), O.gaussian(seed + 2, out_f)


@needs_ref
@pytest.mark.parametrize(("rows", "in_f", "out_f"), [(1, 32, 1), (7, 64, 19), (65, 256, 48)])
def test_linear_q8_and_q4_match_reference(rows, in_f, out_f):
    """quant.hpp:143-169, 355-403 compiled from the reference against the oracle, bit for bit."""
    x, q, s, b = q8_linear_case(3, rows, in_f, out_f)
    for bias in (None, b):
        want = O.linear_q8(O.ref().ref_linear_q8, x, q, s, bias)
        assert O.linear_q8(O.oracle().orc_linear_q8, x, q, s, bias).tobytes() == want.tobytes()
    w = O.gaussian(9, out_f, in_f, scale=0.05)
    pa, sa = O.quantize_q4_0(O.oracle().orc_quantize_q4_0, w)
    pb, sb = O.quantize_q4_0(O.ref().ref_quantize_q4_0, w)
    assert pa.tobytes() == pb.tobytes() and sa.tobytes() == sb.tobytes()
    assert O.unpack_q4_0(O.oracle().orc_unpack_q4_0, pa).tobytes() == O.unpack_q4_0(O.ref().ref_unpack_q4_0, pa).tobytes()
    packed, scales = pa.reshape(out_f, in_f // 2), sa.reshape(out_f, in_f // 32)
    assert (O.linear_q4(O.oracle().orc_linear_q4, x, packed, scales, b).tobytes()
            == O.linear_q4(O.ref().ref_linear_q4, x, packed, scales, b).tobytes())


def test_linear_q8_closed_form_on_the_integer_grid():
    """With x and w already on their Q8_0 grids (values k d, one |k| = 127 per block) every block sum is an exact
    integer and the output is the float64 sum of scaled integer dots (quant.hpp:143-169 by hand)."""
    rng = np.random.default_rng(2)
    kx = rng.integers(-127, 128, size=(3, 64)).astype(np.float32)
    kw = rng.integers(-127, 128, size=(5, 64)).astype(np.float32)
    kx[:, ::32] = 127.0
    kw[:, ::32] = -127.0
    dx, dw = np.float32(0.5), np.float32(0.125)
    x = kx * dx
    q, s = O.quantize_q8_0(O.oracle().orc_quantize_q8_0, kw * dw)
    assert np.all(s == dw)
    out = O.linear_q8(O.oracle().orc_linear_q8, x, q.reshape(5, 64), s.reshape(5, 2))
    for r in range(3):
        for n in range(5):
            acc = 0.0
            for b in range(2):
                isum = int(np.dot(kx[r, 32 * b:32 * b + 32].astype(np.int64), kw[n, 32 * b:32 * b + 32].astype(np.int64)))
                acc += (float(dx) * float(dw)) * float(isum)
            assert out[r, n] == np.float32(acc)


def test_q4_0_packs_two_values_per_byte():
    """Values on the Q4_0 grid (k d, |k| <= 7, one |k| = 7 per block) pack as k + 8 in nibbles and unpack to k."""
    rng = np.random.default_rng(4)
    k = rng.integers(-7, 8, size=(4, 32)).astype(np.float32)
    k[:, 3] = 7.0
    packed, scales = O.quantize_q4_0(O.oracle().orc_quantize_q4_0, (k * np.float32(0.5)).ravel())
    assert np.all(scales == np.float32(0.5))
    assert np.array_equal(O.unpack_q4_0(O.oracle().orc_unpack_q4_0, packed).astype(np.float32), k.ravel())
    assert packed[0] == (int(k[0, 0]) + 8) | ((int(k[0, 16]) + 8) << 4)


# ---- encoder and T5 kernels ----

ERF_POINTS = [0.0, -0.0, 1e-300, 0.3, -0.3, 1.0, 2.4999999, 2.5, -2.5, 3.7, 6.0, 6.0000001, -7.0, 27.3, 27.31, 30.0,
              -30.0, 1e-5, float("inf"), float("-inf"), float("nan")]


@needs_ref
def test_erf_and_erfc_match_reference_and_mathematics():
    o, r = O.oracle_encoder(), O.ref_encoder()
    pts = ERF_POINTS + list(np.linspace(-8, 8, 1001))
    for x in pts:
        for name in ("erf", "erfc"):
            a, b = getattr(o, name)(x), getattr(r, name)(x)
            assert np.float64(a).tobytes() == np.float64(b).tobytes(), (name, x)
    for x in np.linspace(-5.5, 5.5, 221):
        assert math.isclose(o.erf(x), math.erf(x), rel_tol=1e-13, abs_tol=1e-15)
        assert math.isclose(o.erfc(x), math.erfc(x), rel_tol=1e-11, abs_tol=1e-300)


@needs_ref
def test_gelu_and_gelu_backward_match_reference():
    o, r = O.oracle_encoder(), O.ref_encoder()
    x = np.concatenate([O.gaussian(41, 3000, scale=3.0),
                        np.array([0.0, -0.0, 40.0, -40.0, 1e-30, np.inf, -np.inf, np.nan], np.float32)])
    dy = O.gaussian(42, x.size)
    same = lambda a, b: np.array_equal(np.isnan(a), np.isnan(b)) and np.where(np.isnan(a), 0, a).tobytes() == np.where(
        np.isnan(b), 0, b).tobytes()
    assert same(o.gelu(x), r.gelu(x))
    assert same(o.gelu_backward(x, dy), r.gelu_backward(x, dy))


@needs_ref
@pytest.mark.parametrize(("rows", "dim"), [(1, 8), (9, 48), (33, 768)])
def test_layer_norm_and_backward_match_reference(rows, dim):
    o, r = O.oracle_encoder(), O.ref_encoder()
    x, w, b, dy = O.gaussian(1, rows, dim, scale=2.0), O.gaussian(2, dim), O.gaussian(3, dim), O.gaussian(4, rows, dim)
    assert o.layer_norm(x, w, b).tobytes() == r.layer_norm(x, w, b).tobytes()
    for got, want in zip(o.layer_norm_backward(x, w, dy, 1e-6), r.layer_norm_backward(x, w, dy, 1e-6)):
        assert got.tobytes() == want.tobytes()


def test_layer_norm_backward_finite_differences():
    """dx, dw, db of layer_norm against central differences of sum(layer_norm * dy) (float64 tolerance)."""
    o = O.oracle_encoder()
    x, w, b, dy = O.gaussian(5, 3, 16, scale=2.0), O.gaussian(6, 16), O.gaussian(7, 16), O.gaussian(8, 3, 16)
    dx, dw, db = o.layer_norm_backward(x, w, dy, 1e-5)

    def f(xx, ww, bb):  # float64 layer_norm
        xx = xx.astype(np.float64)
        mean = xx.mean(axis=1, keepdims=True)
        inv = 1.0 / np.sqrt(((xx - mean) ** 2).mean(axis=1, keepdims=True) + 1e-5)
        return float(np.sum(((xx - mean) * inv * ww + bb) * dy.astype(np.float64)))

    h = 1e-4
    for k, grad in enumerate((dx, dw, db)):
        base = [a.astype(np.float64) for a in (x, w, b)]
        flat = base[k].ravel()
        for idx in (0, flat.size // 2, flat.size - 1):
            plus, minus = [a.copy() for a in base], [a.copy() for a in base]
            plus[k].ravel()[idx] += h
            minus[k].ravel()[idx] -= h
            numeric = (f(*plus) - f(*minus)) / (2 * h)
            assert math.isclose(grad.ravel()[idx], numeric, rel_tol=1e-3, abs_tol=1e-4)


@needs_ref
@pytest.mark.parametrize(("q_len", "kv_len", "heads", "hd", "vd"), [(5, 7, 2, 8, 8), (17, 17, 4, 16, 12), (1, 3, 1, 4, 4),
                                                                    (3, 0, 2, 4, 4)])
def test_biased_attention_and_backward_match_reference(q_len, kv_len, heads, hd, vd):
    o, r = O.oracle_encoder(), O.ref_encoder()
    q, k, v = O.gaussian(11, q_len, heads, hd), O.gaussian(12, kv_len, heads, hd), O.gaussian(13, kv_len, heads, vd)
    bias, dout = O.gaussian(14, heads, q_len, kv_len, scale=3.0), O.gaussian(15, q_len, heads, vd)
    assert o.biased_attention(q, k, v, bias, 0.25).tobytes() == r.biased_attention(q, k, v, bias, 0.25).tobytes()
    assert o.biased_attention_weights(q, k, bias, 0.25).tobytes() == r.biased_attention_weights(q, k, bias, 0.25).tobytes()
    for got, want in zip(o.biased_attention_backward(q, k, v, bias, dout, 0.25),
                         r.biased_attention_backward(q, k, v, bias, dout, 0.25)):
        assert got.tobytes() == want.tobytes()
