"""GPU parity: every kernel entry point of the C ABI (through etalii_dllm_amd.kernels) against the CPU oracle, bit for
bit, on seeded ordinary and adversarial inputs and the reference tests' edge cases (ignored targets, ragged and
single rows, windows, soft-caps, offsets, errors)."""

from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    from etalii_dllm_amd import kernels

    return kernels


@pytest.fixture(scope="module")
def ora():
    return O.oracle_kernels()


def adversarial(seed: int, *shape: int) -> np.ndarray:
    values = O.gaussian(seed, *shape).astype(np.float64)
    exponents = O.gaussian(seed + 1000, *shape).astype(np.float64)
    out = values * np.power(10.0, np.clip(np.round(exponents * 8), -30, 20))
    out[np.abs(O.gaussian(seed + 2000, *shape)) < 0.05] = 0.0
    return out.astype(np.float32)


def assert_same(a, b, what=""):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    if a.tobytes() != b.tobytes():
        diff = np.flatnonzero(a.view(np.uint32).ravel() != b.view(np.uint32).ravel()) if a.dtype == np.float32 else []
        raise AssertionError(f"{what}: {len(diff)} of {a.size} elements differ, first at {diff[:5]}")


# (8192, 64, 1536): a forward of 768 tiles of 128 x 128 (more than one round of the 512 workgroup slots)
@pytest.mark.parametrize(("rows", "inf", "outf"),
                         [(1, 37, 19), (7, 64, 259), (64, 128, 256), (130, 96, 64), (8192, 64, 1536)])
@pytest.mark.parametrize("kind", ["gaussian", "adversarial"])
def test_linear_forward_and_backward(K, ora, rows, inf, outf, kind):
    make = adversarial if kind == "adversarial" else O.gaussian
    x, w, b, dy = make(1, rows, inf), make(2, outf, inf), make(3, outf), make(4, rows, outf)
    assert_same(K.linear(x, w, b), ora.linear(x, w, b), "linear+bias")
    assert_same(K.linear(x, w), ora.linear(x, w), "linear")
    for got, want, name in zip(K.linear_backward(x, w, dy, True), ora.linear_backward(x, w, dy, True),
                               ("dx", "dw", "db")):
        assert_same(got, want, name)
    dx, dw, db = K.linear_backward(x, w, dy)
    assert db is None


def test_linear_rows_are_batch_invariant(K):
    """The bits of a row of linear / dx do not depend on how many rows are computed with it (M swept)."""
    w, dyw = O.gaussian(5, 300, 160), O.gaussian(6, 300, 160)
    x_all, dy_all = O.gaussian(7, 2048, 160), O.gaussian(8, 2048, 300)
    full = K.linear(x_all, w)
    dfull = K.linear_backward(x_all, dyw, dy_all)[0]
    for m in (1, 7, 64):
        assert_same(K.linear(x_all[:m], w), full[:m], f"linear M={m}")
        assert_same(K.linear_backward(x_all[:m], dyw, dy_all[:m])[0], dfull[:m], f"dx M={m}")


def test_linear_dx_of_an_operand_past_4_gib(K, ora):
    """dX of the head at c3's batch: dy [8192, 151936] is 4.98 GB, read transposed by the matrix-core kernel, whose
    32-bit per-lane copy offsets are taken from each workgroup's own rows (taken from the operand's start they wrapped
    past 2^32 bytes, from row 7065 on). Rows on both sides of that boundary and the last rows against the oracle, and
    the first rows against a 64-row call (batch invariance)."""
    rows, inf, outf = 8192, 1536, 151936
    rng = np.random.default_rng(71)  # 1.2 G values: numpy's generator rather than the reference's serial one
    x = rng.standard_normal((rows, inf), dtype=np.float32)
    w = rng.standard_normal((outf, inf), dtype=np.float32) * np.float32(0.02)
    dy = rng.standard_normal((rows, outf), dtype=np.float32) * np.float32(1e-4)
    dx, _, _ = K.linear_backward(x, w, dy)
    small, _, _ = K.linear_backward(x[:64], w, dy[:64])
    assert_same(dx[:64], small, "rows 0-63 against a 64-row call")
    for sel in ([7063, 7064, 7065, 7066], [8190, 8191]):
        want, _, _ = ora.linear_backward(np.ascontiguousarray(x[sel]), w, np.ascontiguousarray(dy[sel]))
        assert_same(dx[sel], want, f"rows {sel}")


@pytest.mark.parametrize(("rows", "dim"), [(1, 8), (9, 48), (33, 576), (5, 1536)])
def test_rms_norm_forward_and_backward(K, ora, rows, dim):
    x, w, dy = O.gaussian(5, rows, dim, scale=3.0), O.gaussian(6, dim), O.gaussian(7, rows, dim)
    assert_same(K.rms_norm(x, w, 1e-5), ora.rms_norm(x, w, 1e-5), "rms_norm")
    assert_same(K.rms_norm(x, w, 1e-6, True), ora.rms_norm(x, w, 1e-6, True), "rms_norm unit offset")
    assert_same(K.rms_norm(x, None, 1e-6), ora.rms_norm(x, None, 1e-6), "rms_norm no weight")
    for got, want, name in zip(K.rms_norm_backward(x, w, dy, 1e-5), ora.rms_norm_backward(x, w, dy, 1e-5),
                               ("dx", "dw")):
        assert_same(got, want, name)
    for got, want, name in zip(K.rms_norm_backward(x, w, dy, 1e-6, True),
                               ora.rms_norm_backward(x, w, dy, 1e-6, True), ("dx unit", "dw unit")):
        assert_same(got, want, name)


# The column sums' workgroup widths (16, 8 or 4 columns by the rows and columns of the launch): long windows with
# widths whose last workgroup is partial (dims multiples of 4, not of 8 or 16), so the copies clamp, against the
# oracle: the norm weight's dw and a bias gradient (db).
@pytest.mark.parametrize(("rows", "dim"), [(4100, 36), (4099, 100), (2048, 1540), (5000, 4)])
def test_column_sums_at_every_workgroup_width(K, ora, rows, dim):
    x, w, dy = O.gaussian(11, rows, dim, scale=2.0), O.gaussian(12, dim), O.gaussian(13, rows, dim)
    for got, want, name in zip(K.rms_norm_backward(x, w, dy, 1e-6), ora.rms_norm_backward(x, w, dy, 1e-6),
                               ("dx", "dw")):
        assert_same(got, want, f"rms_norm_backward {name}")
    x8, wl = O.gaussian(14, rows, 8), O.gaussian(15, dim, 8, scale=0.1)  # db sums dy's dim columns
    got = K.linear_backward(x8, wl, dy, with_bias=True)
    want = ora.linear_backward(x8, wl, dy, with_bias=True)
    for g, e, name in zip(got, want, ("dx", "dw", "db")):
        assert_same(g, e, f"linear_backward {name}")


@pytest.mark.parametrize(("rotary", "theta"), [(16, 1e6), (8, 1e4), (128, 1e6)])
@pytest.mark.parametrize("interleaved", [False, True])
def test_rope(K, ora, rotary, theta, interleaved):
    hd = max(16, rotary)
    x = O.gaussian(9, 11, 3, hd)
    pos = np.arange(11, dtype=np.int64) * 131
    inv = O.rope_inv_freq(rotary, theta)
    for inverse in (False, True):
        assert_same(K.rope(x, pos, inv, interleaved, inverse), ora.rope(x, pos, inv, interleaved, inverse),
                    f"rope inverse={inverse}")


# Head counts past four rows per wave (the in-kernel cos/sin path batches four heads' loads), partial rotary, and a
# 256-wide head (rows of 128 elements: the table path).
@pytest.mark.parametrize(("heads", "hd", "rotary"), [(14, 64, 64), (2, 64, 64), (7, 128, 128), (9, 96, 32), (5, 80, 64),
                                                     (4, 256, 256), (17, 16, 16)])
@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_many_heads(K, ora, heads, hd, rotary, interleaved):
    x = O.gaussian(10, 37, heads, hd)
    pos = (np.arange(37, dtype=np.int64) * 977) % 5003
    inv = O.rope_inv_freq(rotary, 1e6)
    for inverse in (False, True):
        assert_same(K.rope(x, pos, inv, interleaved, inverse), ora.rope(x, pos, inv, interleaved, inverse),
                    f"rope heads={heads} hd={hd} rotary={rotary} inverse={inverse}")


@pytest.mark.parametrize(("q_len", "kv_len", "heads", "kvh", "hd", "window", "softcap", "offset", "causal"), [
    (9, 9, 6, 2, 8, 0, 0.0, 0, True),
    (5, 9, 6, 2, 8, 0, 0.0, 4, True),
    (9, 9, 6, 3, 8, 3, 0.0, 0, True),
    (9, 9, 4, 4, 8, 0, 0.7, 0, True),
    (130, 130, 4, 2, 64, 0, 0.0, 0, True),
    (70, 70, 2, 1, 128, 17, 0.0, 0, True),
    (70, 70, 6, 2, 12, 0, 0.0, 0, False),  # every key visible (matrix-core tiles)
    (33, 33, 4, 4, 6, 5, 0.0, 0, False),  # non-causal window (row kernels)
    (65, 65, 3, 1, 5, 0, 0.0, 0, True),  # head_dim not a multiple of 4 (row kernels)
    (4, 3000, 4, 2, 16, 0, 0.0, 2996, True),  # past 2048 keys: staged in device memory
    (2100, 2100, 2, 1, 8, 0, 0.5, 0, True),  # soft-capped, past 2048 keys
    (2300, 2300, 4, 2, 16, 0, 0.0, 0, True),  # past 2048 keys on the tiles
])
def test_attention_forward_and_backward(K, ora, q_len, kv_len, heads, kvh, hd, window, softcap, offset, causal):
    """Both paths of the C-ABI attention against the oracle, bit for bit: the training step's matrix-core tiles for
    self-attention shapes, the row kernels for the rest (cached prefix, soft-cap, odd head_dim, non-causal windows),
    including key lengths past the row kernels' LDS staging."""
    q, k, v = O.gaussian(12, q_len, heads, hd), O.gaussian(13, kv_len, kvh, hd), O.gaussian(14, kv_len, kvh, hd)
    dout = O.gaussian(15, q_len, heads, hd)
    scale = 1.0 / np.sqrt(hd)
    assert_same(K.attention(q, k, v, scale, causal, offset, window, softcap),
                ora.attention(q, k, v, scale, causal, offset, window, softcap), "attention")
    got = K.attention_backward(q, k, v, dout, scale, causal, offset, window, softcap)
    want = ora.attention_backward(q, k, v, dout, scale, causal, offset, window, softcap)
    for g, w, name in zip(got, want, ("dq", "dk", "dv")):
        assert_same(g, w, name)


def test_elementwise(K, ora):
    g, up = O.gaussian(8, 5000, scale=6.0), O.gaussian(11, 5000)
    g[:8] = [0.0, -0.0, 40.0, -40.0, 800.0, -800.0, 1e-30, -1e-30]
    assert_same(K.silu(g), ora.silu(g), "silu")
    assert_same(K.swiglu(g, up), ora.swiglu(g, up), "swiglu")
    assert_same(K.silu_backward(g, up), ora.silu_backward(g, up), "silu_backward")
    assert_same(K.gelu_tanh(g), O.gelu_tanh(g), "gelu_tanh")
    assert_same(K.swiglu(g, up, 2), O.gelu_tanh(g) * up, "swiglu kind 2 (gelu_tanh, rounded, then the multiply)")
    with pytest.raises(ValueError, match="kind"):
        K.swiglu(g, up, 1)


@pytest.mark.parametrize(("rows", "vocab"), [(6, 301), (3, 5000), (2, 49152), (6, 1024), (5, 515), (9, 2049),
                                             (6, 151936)])
def test_cross_entropy(K, ora, rows, vocab):
    """Row counts that do and do not fill the 4-row waves; vocabularies of whole 512-column chunks, a partial last
    chunk, one that is not a multiple of 4 (the scalar loads) and the full 151936."""
    logits = O.gaussian(16, rows, vocab, scale=4.0)
    targets = np.array([3, -1, vocab - 1, 0, 17, 17, 5, -1, 2][:rows], np.int64)
    la, da = K.cross_entropy(logits, targets, 0.25)
    lb, db = ora.cross_entropy(logits, targets, 0.25)
    assert la == lb
    assert_same(da, db, "dlogits")


def test_cross_entropy_rejects_target_out_of_range(K):
    with pytest.raises(ValueError, match="target out of range"):
        K.cross_entropy(O.gaussian(1, 2, 10), np.array([1, 10], np.int64))


def test_embedding_backward(K, ora):
    dy, tokens = O.gaussian(17, 12, 5), np.array([3, 1, 3, 0, 3, 1, 9, 9, 9, 2, 0, 3], np.int64)
    assert_same(K.embedding_backward(dy, tokens, 10), ora.embedding_backward(dy, tokens, 10), "embedding")
    with pytest.raises(ValueError, match="out of range"):
        K.embedding_backward(dy, np.array([10] + [0] * 11, np.int64), 10)


def test_sum_squares_and_adamw(K, ora):
    g = adversarial(18, 100003)
    assert K.sum_squares(g) == ora.sum_squares(g)
    p, grad = O.gaussian(18, 3000), O.gaussian(19, 3000)
    m, v = O.gaussian(20, 3000, scale=0.1), np.abs(O.gaussian(21, 3000, scale=0.1))
    pa, ma, va = p.copy(), m.copy(), v.copy()
    pb, mb, vb = p.copy(), m.copy(), v.copy()
    args = (1e-3, 0.9, 0.999, 1e-8, 0.01, 1 - 0.9**3, 1 - 0.999**3, 0.5)
    K.adamw_step(pa, grad, ma, va, *args)
    ora.adamw_step(pb, grad, mb, vb, *args)
    assert_same(pa, pb, "param")
    assert_same(ma, mb, "m")
    assert_same(va, vb, "v")


def sum_squares_cases():
    """Adversarial inputs for the exact parallel sum of squares: binade crossings at every scale, exact round-half-even
    ties of both parities (x = odd * 2^-26 while the sum is in [2, 4): x^2 / ulp ends in .5), leading zeros, a huge
    first element then tiny ones, monotone ramps, and non-finite values."""
    n = 3 * 8192 + 77
    g = O.gaussian(40, n)
    cases = {"gaussian": g, "small": g * np.float32(1e-20), "adversarial": adversarial(41, n)}
    odd = (2 * (np.arange(n) % 4096) + 1).astype(np.float32) * np.float32(2.0 ** -26)
    ties = odd.copy()
    ties[0] = np.float32(1.5)  # s = 2.25 after the first element
    cases["ties"] = ties
    cases["ties_late"] = np.concatenate([np.zeros(5000, np.float32), ties])
    ramp = np.float32(2.0) ** (np.linspace(-60, 60, n).astype(np.float32))
    cases["ramp_up"] = ramp
    cases["ramp_down"] = ramp[::-1].copy()
    cases["huge_then_tiny"] = np.concatenate([[np.float32(3e18)], g * np.float32(1e-12)]).astype(np.float32)
    z = np.zeros(20000, np.float32)
    z[-3:] = [0.5, -0.25, 3.0]
    cases["zeros"] = z
    cases["all_zero"] = np.zeros(9000, np.float32)
    inf_case = g.copy()
    inf_case[9000] = np.inf
    cases["inf"] = inf_case
    nan_case = g.copy()
    nan_case[17000] = np.nan
    cases["nan"] = nan_case
    cases["one"] = np.array([3.0], np.float32)
    # sizes where most blocks are regular and the irregular ones take the 2048-element runs of the walk
    cases["gaussian_2M"] = O.gaussian(42, 2_000_003)
    rows = np.zeros((3000, 1024), np.float32)
    picked = np.unique((O.gaussian(43, 400) * 700 + 1500).astype(np.int64) % 3000)
    rows[picked] = O.gaussian(44, picked.size, 1024)
    cases["sparse_rows"] = rows.ravel()
    long_ties = np.tile(odd, 40)
    long_ties[0] = np.float32(1.5)
    cases["ties_long"] = long_ties
    late = np.zeros(1_500_000 + 40_000, np.float32)
    late[1_500_003:] = O.gaussian(45, 40_000 - 3)
    late[1_500_001] = np.float32(-0.0)
    cases["zeros_then_gaussian"] = late
    cases["all_zero_big"] = np.zeros(300_001, np.float32)
    return cases


@pytest.mark.parametrize("name", sorted(sum_squares_cases()))
def test_exact_parallel_sum_squares_matches_the_serial_chain(K, ora, name):
    values = sum_squares_cases()[name]
    got, want = K.sum_squares(values), ora.sum_squares(values)
    assert np.float64(got).tobytes() == np.float64(want).tobytes(), (name, got, want)


@pytest.mark.parametrize("name", sorted(O.q8_0_cases()))
def test_quantize_and_dequantize_q8_0(K, ora, name):
    x = O.q8_0_cases()[name].reshape(-1, 64)
    q, s = K.quantize_q8_0(x)
    qo, so = O.quantize_q8_0(O.oracle().orc_quantize_q8_0, x)
    assert_same(q.ravel(), qo, "values")
    assert_same(s.ravel(), so, "scales")
    assert_same(K.dequantize_q8_0(q, s).ravel(), O.dequantize_q8_0(qo, so), "dequantized")


@pytest.mark.parametrize(("out_f", "in_f", "rank"), [(48, 32, 2), (64, 96, 16), (130, 257, 3), (8, 12, 4)])
def test_lora_merge_and_adapter_gradients(K, ora, out_f, in_f, rank):
    w, a, b = O.gaussian(61, out_f, in_f), O.gaussian(62, rank, in_f, scale=0.5), O.gaussian(63, out_f, rank)
    g = adversarial(64, out_f, in_f)
    assert_same(K.lora_merge(w, a, b, 2.0), O.lora_merge(ora, w, a, b, 2.0), "merge")
    for got, want, name in zip(K.lora_adapter_gradients(g, a, b, 2.0), O.adapter_gradients(ora, g, a, b, 2.0),
                               ("dA", "dB")):
        assert_same(got, want, name)


@pytest.mark.parametrize("rows,experts,k", [(1, 4, 1), (37, 8, 2), (300, 64, 8), (5, 128, 4), (9, 200, 6), (6, 300, 3)])
@pytest.mark.parametrize("normalize", [False, True])
def test_moe_route_and_backward(K, ora, rows, experts, k, normalize):
    """nn.hpp:864-896 and grad.hpp:507-541: Gaussian logits plus rows of exact ties (the lower expert wins) and a row
    of one large logit; with and without the load-balancing loss's dprobabilities."""
    logits = O.gaussian(rows * 7 + experts, rows, experts, scale=2.0)
    if rows > 2:
        logits[1] = 0.5  # every probability equal
        logits[2, ::2] = logits[2, 1::2]  # pairs of equal probabilities
    logits[0, experts // 2] = 40.0
    if rows > 5:
        logits[3, 0] = np.nan  # NaN first logit: a NaN maximum, every probability NaN (the first experts win)
        logits[4, experts - 1] = np.nan  # NaN last logit: a NaN total, every probability NaN
        logits[5, : experts // 2] = -np.inf
    ia, wa = K.moe_route(logits, k, normalize)
    ib, wb = ora.moe_route(logits, k, normalize)
    assert ia.tobytes() == ib.tobytes()
    assert_same_or_nan(wa, wb, "weights")
    dw = O.gaussian(rows + 3, rows, k)
    dp = O.gaussian(rows + 4, rows, experts, scale=1e-2)
    assert_same_or_nan(K.moe_route_backward(logits, ia, dw, dp, normalize),
                       ora.moe_route_backward(logits, ib, dw, dp, normalize), "dlogits")
    assert_same_or_nan(K.moe_route_backward(logits, ia, dw, None, normalize),
                       ora.moe_route_backward(logits, ib, dw, None, normalize), "dlogits without dprobabilities")


def test_moe_route_rejects_bad_k(K):
    with pytest.raises(ValueError):
        K.moe_route(np.zeros((2, 4), np.float32), 5, False)
    with pytest.raises(ValueError):
        K.moe_route_backward(np.zeros((2, 4), np.float32), np.zeros((2, 1), np.int64), np.zeros((2, 2), np.float32),
                             None, False)


def test_gelu_tanh_and_softcap_backward(K):
    x = np.concatenate([O.gaussian(41, 3000, scale=3.0), adversarial(42, 1000),
                        np.array([0.0, -0.0, 20.0, -20.0, 1e4, np.inf, -np.inf, np.nan], np.float32)])
    dy = O.gaussian(43, x.size)

    def same_up_to_nan_bits(a, b, what):  # a NaN the hardware generates has no defined sign or payload
        nan = np.isnan(a)
        assert np.array_equal(nan, np.isnan(b)), what
        assert_same(np.where(nan, 0, a), np.where(nan, 0, b), what)

    same_up_to_nan_bits(K.gelu_tanh_backward(x, dy), O.gelu_tanh_backward(x, dy), "gelu_tanh_backward")
    for cap in (30.0, 50.0, 0.5):
        same_up_to_nan_bits(K.softcap_backward(x, dy, cap), O.softcap_backward(x, dy, cap), f"softcap {cap}")
    with pytest.raises(ValueError):
        K.softcap_backward(x, dy, 0.0)
    # the forward soft-cap and the elementwise sigmoid (kernels.cpp:629-630, 650-660)
    for cap in (30.0, 0.05):
        same_up_to_nan_bits(K.softcap(x, cap), O.softcap(x, cap), f"softcap forward {cap}")
    same_up_to_nan_bits(K.sigmoid_elementwise(x), O.sigmoid_elementwise(x), "sigmoid_elementwise")
    with pytest.raises(ValueError):
        K.softcap(x, -1.0)


def test_softmax_column_mean_and_dot(K, ora):
    logits = O.gaussian(44, 9, 301, scale=4.0)
    logits[3] = 1.5
    for row in logits:
        assert_same(K.softmax(row), ora.softmax(row.copy()), "softmax")
    assert_same(K.softmax(logits), np.stack([ora.softmax(r.copy()) for r in logits]), "softmax rows")
    x = adversarial(45, 1000, 7)
    assert_same(K.column_mean(x), ora.column_mean(x), "column_mean")
    a, b = adversarial(46, 5000), O.gaussian(47, 5000)
    assert K.dot(a, b) == ora.dot(a, b)


@pytest.mark.parametrize("rows", [1, 2, 3, 5, 15, 17, 33])
def test_linear_matrix_core_tails_and_non_finite(K, ora, rows):
    """Reductions of every length mod 16 through the matrix-core path (K and N multiples of 4), with infinities and
    NaNs in the operands: the padded steps of a partial stage must leave every sum's bits alone."""
    x, w, dy = adversarial(11, rows, 64), adversarial(12, 128, 64), adversarial(13, rows, 128)
    for got, want, name in zip(K.linear_backward(x, w, dy), ora.linear_backward(x, w, dy), ("dx", "dw", "db")):
        if want is not None:
            assert_same(got, want, f"{name} rows={rows}")
    x[0, 3] = np.inf
    dy[rows - 1, 5] = np.nan
    w[7, 9] = -np.inf
    pairs = list(zip(K.linear_backward(x, w, dy)[:2], ora.linear_backward(x, w, dy)[:2], ("dx", "dw")))
    pairs.append((K.linear(x, w), ora.linear(x, w), "linear"))
    for got, want, name in pairs:
        got, want = np.asarray(got), np.asarray(want)
        nan = np.isnan(want)  # a NaN the hardware generates has no defined sign or payload
        assert np.array_equal(np.isnan(got), nan), f"{name} rows={rows}: NaN positions"
        assert_same(np.where(nan, 0, got), np.where(nan, 0, want), f"{name} rows={rows} non-finite")


def q8_case(seed: int, rows: int, in_f: int, out_f: int):
    x = O.gaussian(seed, rows, in_f)
    x[0, :32] = 0.0
    if rows > 2:
        x[2, 5] = np.inf
        x[2, 40 % in_f] = -7e30
    w = O.gaussian(seed + 1, out_f, in_f, scale=0.02)
    q, s = O.quantize_q8_0(O.oracle().orc_quantize_q8_0, w)
    return x, q.reshape(out_f, in_f), s.reshape(out_f, in_f // 32), O.gaussian(seed + 2, out_f)


@pytest.mark.parametrize(("rows", "in_f", "out_f"), [(1, 32, 1), (7, 64, 19), (8, 8960, 37), (9, 96, 40), (2, 8192 + 32, 5), (65, 256, 48), (130, 1024, 200)])
def test_linear_q8_and_q4(K, rows, in_f, out_f):
    """Q8_0 / Q4_0 linear (quant.hpp:143-169, 355-403) on the int8 matrix cores against the oracle, bit for bit."""
    x, q, s, b = q8_case(5, rows, in_f, out_f)
    for bias in (None, b):
        assert_same(K.linear_q8(x, q, s, bias), O.linear_q8(O.oracle().orc_linear_q8, x, q, s, bias), "linear_q8")
    w = O.gaussian(9, out_f, in_f, scale=0.05)
    w[0, 3] = np.nan
    packed, scales = K.quantize_q4_0(w)
    want_p, want_s = O.quantize_q4_0(O.oracle().orc_quantize_q4_0, w)
    assert packed.view(np.uint8).tobytes() == want_p.tobytes() and scales.tobytes() == want_s.tobytes()
    assert_same(K.unpack_q4_0(packed), O.unpack_q4_0(O.oracle().orc_unpack_q4_0, want_p).reshape(out_f, in_f),
                "unpack_q4_0")
    assert_same(K.linear_q4(x, packed, scales, b),
                O.linear_q4(O.oracle().orc_linear_q4, x, want_p.reshape(out_f, in_f // 2), want_s.reshape(out_f, -1), b),
                "linear_q4")


def test_linear_q8_rows_are_batch_invariant(K):
    x, q, s, _ = q8_case(7, 300, 128, 96)
    full = K.linear_q8(x, q, s)
    for m in (1, 7, 64):
        assert_same(K.linear_q8(x[:m], q, s), full[:m], f"linear_q8 M={m}")


def assert_same_or_nan(a, b, what=""):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a)
    assert np.array_equal(nan, np.isnan(b)), f"{what}: NaN positions differ"
    assert_same(np.where(nan, 0, a), np.where(nan, 0, b), what)


def test_gelu_and_backward_match_the_oracle(K):
    """Exact GELU and its gradient (kernels.cpp:631, 877-889), bit for bit, over the erf/erfc branch points and
    non-finite inputs."""
    x = np.concatenate([O.gaussian(11, 4001, scale=3.0),
                        np.array([0, -0.0, 0.5, -0.5, 0.84375, -0.84375, 1.25, -1.25, 2.857, -2.857, 6, -6, 28, -28,
                                  1e-30, -1e-30, 1e-40, np.inf, -np.inf, np.nan, 3e38, -3e38], np.float32)])
    dy = O.gaussian(12, x.size)
    enc = O.oracle_encoder()
    assert_same_or_nan(K.gelu(x), enc.gelu(x), "gelu")
    assert_same_or_nan(K.gelu_backward(x, dy), enc.gelu_backward(x, dy), "gelu_backward")


@pytest.mark.parametrize(("rows", "dim"),
                         [(1, 1), (3, 7), (37, 64), (130, 768), (5, 1031), (70, 20), (1, 4), (300, 1028)])
def test_layer_norm_and_backward_match_the_oracle(K, rows, dim):
    """LayerNorm forward and backward (kernels.cpp:612-625, 858-875), bit for bit."""
    x, w, b, dy = O.gaussian(21, rows, dim), O.gaussian(22, dim), O.gaussian(23, dim), O.gaussian(24, rows, dim)
    enc = O.oracle_encoder()
    for eps in (1e-12, 1e-6):
        assert_same(K.layer_norm(x, w, b, eps), enc.layer_norm(x, w, b, eps), "layer_norm")
        for got, want, what in zip(K.layer_norm_backward(x, w, dy, eps), enc.layer_norm_backward(x, w, dy, eps),
                                   ("dx", "dw", "db")):
            assert_same(got, want, f"layer_norm_backward {what}")


@pytest.mark.parametrize(("q_len", "kv_len", "heads", "hd", "vd"),
                         [(1, 3, 1, 4, 4), (5, 7, 2, 8, 8), (33, 70, 3, 64, 64), (3, 0, 2, 4, 4), (6, 6, 2, 6, 8),
                          (17, 17, 4, 16, 12), (1, 1, 1, 4, 4), (64, 64, 2, 64, 64), (130, 130, 3, 64, 32),
                          (70, 70, 1, 12, 20), (200, 200, 2, 8, 128)])
def test_biased_attention_and_backward_match_the_oracle(K, q_len, kv_len, heads, hd, vd):
    """T5 biased attention forward, weights and backward (kernels.cpp:707-727, 753-773, 961-990), bit for bit, on
    the per-(query, head) kernels (cross-attention shapes, head_dim not a multiple of 4) and the matrix-core tiles
    (self-attention shapes); kv_len 0 is the empty case (zero output and gradients)."""
    q, k, v = O.gaussian(31, q_len, heads, hd), O.gaussian(32, kv_len, heads, hd), O.gaussian(33, kv_len, heads, vd)
    bias, dout = O.gaussian(34, heads, q_len, kv_len), O.gaussian(35, q_len, heads, vd)
    if kv_len > 2:
        bias[0, 0, :2] = -np.inf  # masked keys
    enc = O.oracle_encoder()
    assert_same(K.biased_attention(q, k, v, bias, 0.25), enc.biased_attention(q, k, v, bias, 0.25), "forward")
    if kv_len:
        assert_same(K.biased_attention_weights(q, k, bias, 0.25), enc.biased_attention_weights(q, k, bias, 0.25),
                    "weights")
    for got, want, what in zip(K.biased_attention_backward(q, k, v, bias, dout, 0.25),
                               enc.biased_attention_backward(q, k, v, bias, dout, 0.25),
                               ("dq", "dk", "dv", "dbias")):
        assert_same_or_nan(got, want, f"biased_attention_backward {what}")


def test_elementwise_scalar_tails_and_misaligned_views(K, ora):
    """The 16-byte vector kernels (SwiGLU, AdamW) hand n % 4 tail elements and arrays that are not 16-byte aligned to
    their scalar kernels: n = 5001, and device views starting 4 bytes into an allocation, through the C ABI."""
    import ctypes as C

    n = 5001
    g, up = O.gaussian(51, n, scale=6.0), O.gaussian(52, n)
    assert_same(K.swiglu(g, up), ora.swiglu(g, up), "swiglu n % 4 = 1")
    assert_same(K.silu_backward(g, up), ora.silu_backward(g, up), "silu_backward n % 4 = 1")
    lib, Device = K.lib, K.Device

    def shifted(values):  # a device copy that starts 4 bytes into its allocation
        d = Device(values.nbytes + 16)
        K.check(lib.dllm_hip_upload(C.c_void_p(d.ptr.value + 4), values.ctypes.data, values.nbytes))
        return d, C.c_void_p(d.ptr.value + 4)

    def fetch(p, count):
        out = np.empty(count, np.float32)
        K.check(lib.dllm_hip_download(out.ctypes.data, p, out.nbytes))
        return out

    dg, pg = shifted(g)
    du, pu = shifted(up)
    do, po = shifted(np.zeros(n, np.float32))
    K.check(lib.dllm_hip_swiglu(pg, pu, po, n, 0, None))
    assert_same(fetch(po, n), ora.swiglu(g, up), "swiglu misaligned")
    p, grad = O.gaussian(53, n, scale=0.02), O.gaussian(54, n, scale=1e-3)
    m, v = O.gaussian(55, n, scale=1e-4), np.abs(O.gaussian(56, n, scale=1e-6))
    args = (1e-3, 0.9, 0.999, 1e-8, 0.01, 1 - 0.9 ** 2, 1 - 0.999 ** 2, 0.7)
    dp, pp = shifted(p)
    dgr, pgr = shifted(grad)
    dm, pm = shifted(m)
    dv, pv = shifted(v)
    K.check(lib.dllm_hip_adamw_step(pp, pgr, pm, pv, n, *args, None))
    want_p, want_m, want_v = p.copy(), m.copy(), v.copy()
    ora.adamw_step(want_p, grad, want_m, want_v, *args)
    assert_same(fetch(pp, n), want_p, "adamw param misaligned")
    assert_same(fetch(pm, n), want_m, "adamw m misaligned")
    assert_same(fetch(pv, n), want_v, "adamw v misaligned")
    K.adamw_step(p, grad, m, v, *args)  # aligned, n % 4 = 1
    assert_same(p, want_p, "adamw param n % 4 = 1")
    assert_same(m, want_m, "adamw m n % 4 = 1")
    assert_same(v, want_v, "adamw v n % 4 = 1")


def test_device_copy(K):
    """dllm_hip_copy: whole 16-byte vectors plus a byte tail, and a misaligned pair (the runtime's copy)."""
    import ctypes as C

    for nbytes, offset in ((0, 0), (7, 0), (4096 * 16 + 13, 0), ((1 << 22) + 5, 0), (1000, 4)):
        src = np.frombuffer(np.random.default_rng(nbytes).bytes(nbytes + 16), np.uint8).copy()
        ds, dd = K.Device.of(src), K.Device(nbytes + 16)
        K.check(K.lib.dllm_hip_copy(C.c_void_p(dd.ptr.value + offset), C.c_void_p(ds.ptr.value + offset), nbytes,
                                    None))
        K.check(K.lib.dllm_hip_synchronize())
        got = np.empty(nbytes + 16, np.uint8)
        K.check(K.lib.dllm_hip_download(got.ctypes.data, dd.ptr, got.nbytes))
        assert got[offset:offset + nbytes].tobytes() == src[offset:offset + nbytes].tobytes(), nbytes
