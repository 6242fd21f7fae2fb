"""Pins the NumPy oracle (``oracle/``) before it is trusted as the checker.

Three kinds of evidence, none of which re-types the oracle's own formula:

1. the reference's own quantization tests (``test_enilnets.py:11133-11243``)
   and its MoE dense-mixture oracle (``:8331-8353``), ported as invariants;
2. an independent exact-arithmetic model: Python ``Fraction`` division with
   explicit round-to-nearest-even to float32 / float64, and Python's
   half-even ``round`` for the codes;
3. brute force around the half-way points ``(k + 1/2) * scale``, with
   planted mistakes (reciprocal multiply, round-half-away, a dropped
   ``+ zero_point``, a transposed weight) that must be caught.
"""

from fractions import Fraction

import numpy as np
import pytest

import oracle


# ---------------------------------------------------------------------------
# exact arithmetic helpers (independent of NumPy's ufuncs)
# ---------------------------------------------------------------------------
def round_fraction(q: Fraction, mant_bits: int, emin: int) -> float:
    """Round a rational to the nearest binary float with ``mant_bits``
    significand bits (ties to even); subnormals below ``2**emin``."""
    if q == 0:
        return 0.0
    sign = -1.0 if q < 0 else 1.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp_exp = max(e, emin) - (mant_bits - 1)
    scaled = a / (Fraction(2) ** ulp_exp)
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(Fraction(n) * Fraction(2) ** ulp_exp)


def rn32(q: Fraction) -> float:
    return round_fraction(q, 24, -126)


def rn64(q: Fraction) -> float:
    return round_fraction(q, 53, -1022)


def exact_scale(amax: float, qmax: int, rn) -> float:
    return rn(Fraction(amax) / qmax) if amax > 0 else 1.0


def exact_code(x: float, s: float, rn, qmin=-127, qmax=127) -> float:
    v = rn(Fraction(x) / Fraction(s))
    return float(min(max(round(v), qmin), qmax))


# ---------------------------------------------------------------------------
# 1. the reference's own invariants (test_enilnets.py:11133-11243)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("scheme", ["symmetric", "asymmetric"])
def test_grid_round_trip_half_step(scheme):
    # test_enilnets.py:11133-11145
    x = np.linspace(-3.0, 5.0, 101)
    scale, zp = oracle.compute_scale(np.min(x), np.max(x), 8, scheme)
    q = oracle.quantize(x, scale, zp, 8, scheme)
    assert np.all(q == np.round(q))
    back = oracle.dequantize(q, scale, zp)
    assert float(np.max(np.abs(back - x))) <= float(np.max(scale)) * 0.5 + 1e-9


def test_symmetric_keeps_exact_zeros():
    # test_enilnets.py:11147-11153
    rng = np.random.default_rng(1)
    x = np.concatenate([np.zeros(50), rng.standard_normal(50)])
    q, _, _ = oracle.quantize_tensor(x, bits=8, scheme="symmetric")
    assert np.all(q[:50] == 0)


def test_more_bits_less_error():
    # test_enilnets.py:11155-11160
    x = np.random.default_rng(2).standard_normal(500)
    errors = [float(np.mean(np.abs(oracle.quantize_tensor(x, bits=b)[0] - x)))
              for b in (4, 6, 8, 12)]
    assert errors == sorted(errors, reverse=True)


def test_per_channel_beats_per_tensor():
    # test_enilnets.py:11162-11177
    w = np.random.default_rng(3).standard_normal((8, 16)) * 0.01
    w[0] = w[0] * 1000.0
    pt = oracle.quantize_tensor(w, 8, per_channel=False)[0]
    pc = oracle.quantize_tensor(w, 8, per_channel=True)[0]
    err_pt = float(np.mean(np.abs(pt[1:] - w[1:])))
    err_pc = float(np.mean(np.abs(pc[1:] - w[1:])))
    assert err_pc < err_pt / 50
    assert float(np.mean(np.abs(pc - w))) <= float(np.mean(np.abs(pt - w)))


def _mlp(rng, dtype=np.float32):
    class M:
        pass
    m = M()
    w1 = (rng.standard_normal((32, 20)) * 0.3).astype(dtype)
    w2 = (rng.standard_normal((4, 32)) * 0.3).astype(dtype)
    m.layers = [
        {"type": "dense", "weights": w1, "bias": np.zeros(32, dtype), "activation": "relu",
         "use_bias": True, "activation_params": {}},
        {"type": "dense", "weights": w2, "bias": np.zeros(4, dtype), "activation": "softmax",
         "use_bias": True, "activation_params": {}},
    ]
    return m


def test_quantize_weights_report_and_error():
    # test_enilnets.py:11179-11199
    import copy
    rng = np.random.default_rng(4)
    m = _mlp(rng)
    X = rng.standard_normal((64, 20)).astype(np.float32)
    ref = [oracle.forward(m.layers, X)[-1]]
    errors = {}
    for bits in (8, 4):
        mm = copy.deepcopy(m)
        report = oracle.quantize_weights(mm, bits=bits)
        assert report["bits"] == bits
        assert report["parameters"] == 32 * 20 + 4 * 32
        assert report["compression"] == pytest.approx(32 / bits, abs=1e-6)
        assert report["quantized_bytes"] == report["parameters"] * bits // 8
        errors[bits] = oracle.quantization_error(ref, [oracle.forward(mm.layers, X)[-1]])[
            "relative_error"]
    assert errors[8] < errors[4]
    assert errors[8] < 1e-2


def test_codes_on_grid():
    # test_enilnets.py:11201-11210
    rng = np.random.default_rng(5)
    m = _mlp(rng)
    oracle.quantize_weights(m, bits=8, scheme="symmetric")
    spec = m.layers[0]["quant"]["weights"]
    codes = m.layers[0]["weights"] / spec["scale"]
    assert np.all(np.abs(codes - np.round(codes)) < 1e-4)


def test_quant_range_and_validation():
    # test_enilnets.py:11236-11243
    assert oracle.quant_range(8, "symmetric") == (-127, 127)
    assert oracle.quant_range(8, "asymmetric") == (0, 255)
    assert oracle.quant_range(2, "symmetric") == (-1, 1)
    assert oracle.quant_range(16, "asymmetric") == (0, 65535)
    for bad in ((1, "symmetric"), (17, "symmetric"), (8, "bogus")):
        with pytest.raises(ValueError):
            oracle.quant_range(*bad)


# ---------------------------------------------------------------------------
# 2. exact arithmetic
# ---------------------------------------------------------------------------
def test_symmetric_per_tensor_matches_exact_arithmetic_f32():
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((7, 13)) * 0.05).astype(np.float32)
    fq, scale, zp = oracle.quantize_tensor(w, 8)
    amax = max(abs(float(w.min())), abs(float(w.max())))
    s = exact_scale(amax, 127, rn32)
    assert float(scale) == s
    assert scale.dtype == np.float32 and scale.shape == ()
    assert zp.dtype == np.float32 and float(zp) == 0.0
    for xi, fi in zip(w.reshape(-1), fq.reshape(-1)):
        c = exact_code(float(xi), s, rn32)
        assert float(fi) == rn32(Fraction(c) * Fraction(s))


def test_symmetric_per_channel_matches_exact_arithmetic_f64():
    rng = np.random.default_rng(7)
    w = rng.standard_normal((5, 9)) * 3.0
    fq, scale, _ = oracle.quantize_tensor(w, 8, per_channel=True)
    assert scale.shape == (5, 1) and scale.dtype == np.float64 and fq.dtype == np.float64
    for r in range(5):
        amax = float(np.max(np.abs(w[r])))
        s = exact_scale(amax, 127, rn64)
        assert float(scale[r, 0]) == s
        for xi, fi in zip(w[r], fq[r]):
            c = exact_code(float(xi), s, rn64)
            assert float(fi) == rn64(Fraction(c) * Fraction(s))


def test_asymmetric_matches_exact_arithmetic():
    rng = np.random.default_rng(8)
    w = (rng.uniform(-0.3, 2.0, (4, 6))).astype(np.float32)
    fq, scale, zp = oracle.quantize_tensor(w, 8, "asymmetric")
    low, high = float(w.min()), float(w.max())
    span = rn32(Fraction(high) - Fraction(low))
    s = rn32(Fraction(span) / 255)
    z = float(round(rn32(0 - Fraction(rn32(Fraction(low) / Fraction(s))))))
    assert float(scale) == s and float(zp) == z
    for xi, fi in zip(w.reshape(-1), fq.reshape(-1)):
        v = rn32(Fraction(rn32(Fraction(float(xi)) / Fraction(s))) + Fraction(z))
        c = min(max(round(v), 0), 255)
        assert float(fi) == rn32(Fraction(rn32(Fraction(c) - Fraction(z))) * Fraction(s))


def test_zero_range_gives_unit_scale_and_nan_propagates():
    fq, scale, _ = oracle.quantize_tensor(np.zeros((3, 4), np.float32), 8, per_channel=True)
    assert np.all(scale == 1.0) and np.all(fq == 0)
    w = np.array([1.0, np.nan, -2.0], np.float32)
    fq, scale, _ = oracle.quantize_tensor(w, 8)
    # amax is NaN, NaN > 0 is False -> scale 1 (quantization.py:44)
    assert float(scale) == 1.0
    assert np.isnan(fq[1]) and fq[0] == 1.0 and fq[2] == -2.0


def test_signed_zero_semantics():
    # x / s + 0.0 turns -0.0 into +0.0 before rounding; small negatives
    # still round to -0.0 and dequantize to -0.0.
    s = np.float32(0.1)
    zp = np.float32(0.0)
    q = oracle.quantize(np.array([-0.0, -0.01, 0.01], np.float32), s, zp, 8, "symmetric")
    assert not np.signbit(q[0]) and np.signbit(q[1]) and not np.signbit(q[2])
    f = oracle.dequantize(q, s, zp)
    assert not np.signbit(f[0]) and np.signbit(f[1])


def test_codes_bounds_and_extreme_hit():
    rng = np.random.default_rng(9)
    for _ in range(20):
        w = (rng.standard_normal((16, 33)) * rng.uniform(1e-3, 10)).astype(np.float32)
        codes, scale = oracle.int8_codes(w, per_channel=True)
        assert codes.dtype == np.int8
        assert np.all(np.abs(codes.astype(np.int32)) <= 127)
        assert np.all(np.max(np.abs(codes.astype(np.int32)), axis=1) == 127)


# ---------------------------------------------------------------------------
# 3. brute force at the half-way points, with planted mistakes
# ---------------------------------------------------------------------------
def _halfway_inputs(seed=10, n_scales=12):
    rng = np.random.default_rng(seed)
    xs, ss = [], []
    for _ in range(n_scales):
        s = np.float32(rng.uniform(1e-3, 1.0) / 127)
        for k in range(-127, 127):
            t = np.float32(float((Fraction(k) + Fraction(1, 2)) * Fraction(float(s))))
            x = t
            for _ in range(2):
                x = np.nextafter(x, np.float32(-np.inf))
            for _ in range(5):
                xs.append(x)
                ss.append(s)
                x = np.nextafter(x, np.float32(np.inf))
    return np.array(xs, np.float32), np.array(ss, np.float32)


def _exact_codes(xs, ss):
    return np.array([exact_code(float(x), float(s), rn32) for x, s in zip(xs, ss)], np.float32)


def test_halfway_points_match_exact_rounding():
    xs, ss = _halfway_inputs()
    got = oracle.quantize(xs, ss, np.zeros_like(ss), 8, "symmetric")
    want = _exact_codes(xs, ss)
    assert np.array_equal(got, want)


def test_planted_mistakes_are_caught():
    xs, ss = _halfway_inputs()
    want = _exact_codes(xs, ss)
    # reciprocal multiply instead of division
    recip = np.clip(np.round(xs * (np.float32(1) / ss)), -127, 127)
    # round half away from zero instead of half to even
    away = np.clip(np.trunc(xs / ss + np.copysign(np.float32(0.5), xs / ss)), -127, 127)
    assert not np.array_equal(recip, want)
    assert not np.array_equal(away, want)
    # a dropped "+ zero_point" changes the sign of zero codes
    q = oracle.quantize(np.array([-0.0], np.float32), np.float32(1), np.float32(0), 8,
                        "symmetric")
    assert not np.signbit(q[0]) and np.signbit(np.round(np.float32(-0.0) / np.float32(1)))


# ---------------------------------------------------------------------------
# Dense / W8A8 / MoE / activations
# ---------------------------------------------------------------------------
def test_w8a8_accumulator_is_the_exact_integer_dot():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((5, 40)).astype(np.float32)
    w = rng.standard_normal((7, 40)).astype(np.float32)
    wc, ws = oracle.int8_codes(w)
    y, acc, xs, xc = oracle.w8a8_dense(x, wc, ws)
    for i in range(5):
        for j in range(7):
            exact = sum(int(a) * int(b) for a, b in zip(xc[i], wc[j]))
            assert acc[i, j] == exact
    # a transposed weight is caught
    bad = np.dot(xc.astype(np.float64), wc.astype(np.float64)[:, ::-1].T)
    assert not np.array_equal(bad.astype(np.int32), acc)
    # y is the rescaled accumulator
    want = (acc.astype(np.float64) * xs.astype(np.float64)) * ws.reshape(1, -1).astype(np.float64)
    assert np.allclose(y, want, rtol=1e-6, atol=1e-6)


def test_dense_forward_matches_float64_math():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((9, 31)).astype(np.float32)
    w = (rng.standard_normal((6, 31)) * 0.1).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    layer = {"type": "dense", "weights": w, "bias": b, "activation": "linear"}
    y, z = oracle.dense_forward(layer, x)
    exact = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.max(np.abs(z - exact)) < 1e-5
    layer["activation"] = "relu"
    y, _ = oracle.dense_forward(layer, x)
    assert np.array_equal(y, np.where(z < 0, 0, z))


def test_activation_closed_forms():
    x = np.array([-3.0, -0.5, 0.0, 0.5, 3.0])
    assert np.allclose(oracle.activate("sigmoid", x), 1 / (1 + np.exp(-x)))
    assert oracle.activate("gelu", np.array([0.0]))[0] == 0.0
    g = oracle.activate("gelu", np.array([10.0]))[0]
    assert abs(g - 10.0) < 1e-12
    assert np.allclose(oracle.activate("swish", x), x / (1 + np.exp(-x)))
    assert np.allclose(oracle.activate("softplus", x), np.log1p(np.exp(x)))
    sm = oracle.activate("softmax", np.array([[1.0, 2.0, 3.0]]))
    assert abs(sm.sum() - 1) < 1e-12 and np.all(np.diff(sm[0]) > 0)
    with pytest.raises(ValueError):
        oracle.activate("nope", x)


def _moe_layer(rng, d=6, h=10, e=4, k=2):
    return {"type": "moe", "embed_dim": d, "num_experts": e, "top_k": k,
            "hidden_dim": h, "activation": "gelu",
            "W1": rng.standard_normal((e, h, d)) * 0.3, "b1": rng.standard_normal((e, h)) * 0.1,
            "W2": rng.standard_normal((e, d, h)) * 0.3, "b2": rng.standard_normal((e, d)) * 0.1,
            "Wr": rng.standard_normal((e, d)) * 0.5, "br": np.zeros(e)}


def test_moe_matches_dense_mixture():
    # test_enilnets.py:8331-8353: run every expert on every token and keep
    # the top-k gates; must equal the routed computation in float64.
    rng = np.random.default_rng(13)
    layer = _moe_layer(rng)
    x = rng.standard_normal((3, 5, 6))
    got = oracle.moe_forward(x, layer)
    flat = x.reshape(-1, 6)
    logits = flat @ layer["Wr"].T + layer["br"]
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p = p / p.sum(axis=1, keepdims=True)
    want = np.zeros_like(flat)
    for t in range(flat.shape[0]):
        top = np.argsort(-p[t])[:2]
        for e in range(4):
            h = oracle.activate("gelu", flat[t] @ layer["W1"][e].T + layer["b1"][e])
            y = h @ layer["W2"][e].T + layer["b2"][e]
            if e in top:
                want[t] += p[t, e] * y
    assert np.allclose(got.reshape(-1, 6), want, atol=1e-10, rtol=0)


def test_window_mask_matches_definition():
    # nn/forward.py:102-117 by its definition: key j is hidden from query i
    # when causal and j > i, or when |i - j| > window.
    for causal in (False, True):
        for window in (None, 0, 1, 3):
            m = oracle.window_mask(7, causal, window)
            if not causal and window is None:
                assert m is None
                continue
            for i in range(7):
                for j in range(7):
                    hidden = (causal and j > i) or (window is not None and abs(i - j) > window)
                    assert m[i, j] == (-np.inf if hidden else 0.0)


def _mha_layer(rng, e=8, h=2, hkv=None, causal=False, window=None):
    hkv = h if hkv is None else hkv
    dh = e // h
    layer = {"type": "multihead_attention", "embed_dim": e, "num_heads": h,
             "num_kv_heads": hkv, "head_dim": dh, "causal": causal, "window_size": window}
    for name, rows in (("q", e), ("k", hkv * dh), ("v", hkv * dh), ("o", e)):
        layer["W" + name] = rng.standard_normal((rows, e)) * 0.4
        layer["b" + name] = rng.standard_normal(rows) * 0.1
    return layer


def test_mha_matches_explicit_loops():
    # Per batch, head, query: scores against every allowed key, softmax,
    # weighted sum of values, in plain Python loops over float64.
    rng = np.random.default_rng(21)
    for causal, window, hkv in ((False, None, 2), (True, None, 2), (False, 1, 1), (True, 2, 2)):
        L = _mha_layer(rng, hkv=hkv, causal=causal, window=window)
        x = rng.standard_normal((2, 5, 8))
        got = oracle.mha_forward(x, L)
        q = x @ L["Wq"].T + L["bq"]
        k = x @ L["Wk"].T + L["bk"]
        v = x @ L["Wv"].T + L["bv"]
        dh, H = L["head_dim"], L["num_heads"]
        ctx = np.zeros_like(q)
        for b in range(2):
            for h in range(H):
                g = h // (H // hkv)
                for i in range(5):
                    keys = [j for j in range(5) if not (causal and j > i)
                            and not (window is not None and abs(i - j) > window)]
                    s = np.array([q[b, i, h*dh:(h+1)*dh] @ k[b, j, g*dh:(g+1)*dh]
                                  for j in keys]) / np.sqrt(dh)
                    w = np.exp(s - s.max())
                    w /= w.sum()
                    ctx[b, i, h*dh:(h+1)*dh] = sum(wj * v[b, j, g*dh:(g+1)*dh]
                                                   for wj, j in zip(w, keys))
        want = ctx @ L["Wo"].T + L["bo"]
        assert np.allclose(got, want, atol=1e-12, rtol=0)


def test_mha_window_zero_and_gqa_invariants():
    # test_enilnets.py:7722-7733 (window 0 reduces to Wo(Wv x)) and
    # :7557-7573 (GQA equals MHA with group-major repeated K/V weights).
    rng = np.random.default_rng(22)
    L = _mha_layer(rng, window=0)
    x = rng.standard_normal((2, 5, 8))
    want = (x @ L["Wv"].T + L["bv"]) @ L["Wo"].T + L["bo"]
    assert np.allclose(oracle.mha_forward(x, L), want, atol=1e-12)
    g = _mha_layer(rng, h=4, hkv=2)
    m = dict(g, num_kv_heads=4)
    for w, b in (("Wk", "bk"), ("Wv", "bv")):
        m[w] = np.repeat(g[w].reshape(2, 2, 8), 2, axis=0).reshape(8, 8)
        m[b] = np.repeat(g[b].reshape(2, 2), 2, axis=0).reshape(8)
    assert np.allclose(oracle.mha_forward(x, g), oracle.mha_forward(x, m), atol=1e-12)


def test_layernorm_closed_form():
    # gamma = 1, beta = 0: every row has mean 0 and variance var/(var+eps);
    # a constant row maps to beta.
    rng = np.random.default_rng(23)
    x = rng.standard_normal((4, 3, 16)) * 3 + 1
    L = {"gamma": np.ones(16), "beta": np.zeros(16), "epsilon": 1e-5}
    y = oracle.layernorm_forward(x, L)
    var = x.var(axis=-1)
    assert np.allclose(y.mean(axis=-1), 0, atol=1e-12)
    assert np.allclose(y.var(axis=-1), var / (var + 1e-5), atol=1e-12)
    L2 = {"gamma": np.arange(16.0), "beta": np.full(16, 0.5)}
    assert np.allclose(oracle.layernorm_forward(np.full((2, 16), 7.0), L2), 0.5)


def test_forward_front_end_closed_forms():
    # forward.py:414-422 (embedding: the table rows of the int ids),
    # :597-603 (positional table rows added per
    # position), :398-413 (dropout is the identity at inference)
    table = np.arange(20, dtype=np.float32).reshape(5, 4)
    pe = np.full((8, 4), 0.5, np.float32)
    layers = [{"type": "embedding", "weights": table},
              {"type": "positional_encoding", "pe": pe, "_pos_type": "sinusoidal"},
              {"type": "dropout", "rate": 0.5}]
    out = oracle.forward(layers, np.array([[4, 0, 2]]))
    assert np.array_equal(out[1], table[[[4, 0, 2]]])
    assert np.array_equal(out[2], table[[[4, 0, 2]]] + 0.5)
    assert out[3] is out[2]
    # Forward makes a 1-D input one row first (forward.py:286-287)
    one = oracle.forward(layers[:1], np.array([3, 1]))
    assert one[1].shape == (1, 2, 4) and np.array_equal(one[1][0], table[[3, 1]])


def test_qat_weight_is_per_channel_quantize_tensor():
    # graph/quantization.py:119-130 takes min / max over every axis but 0 and
    # fake-quantizes symmetrically: exactly quantize_tensor(per_channel=True)
    rng = np.random.default_rng(41)
    w = (rng.standard_normal((12, 30)) * 0.2).astype(np.float32)
    fq = oracle.qat_quantized_weight(w, 8, per_channel=True)
    want, _, _ = oracle.quantize_tensor(w, 8, "symmetric", per_channel=True)
    assert fq.dtype == want.dtype and np.array_equal(fq, want)
    fq1 = oracle.qat_quantized_weight(w, 4, per_channel=False)
    want1, _, _ = oracle.quantize_tensor(w, 4, "symmetric", per_channel=False)
    assert np.array_equal(fq1, want1)
    # a planted mistake: statistics over axis 0 instead of axis 1
    wrong = oracle.fake_quantize(w, *oracle.compute_scale(w.min(0, keepdims=True),
                                                          w.max(0, keepdims=True), 8,
                                                          "symmetric"), 8, "symmetric")
    assert not np.array_equal(fq, wrong)


def test_qat_observer_and_ste_mask_closed_forms():
    obs = oracle.MovingRange(momentum=0.5)
    obs.observe(np.array([-1.0, 3.0]))
    obs.observe(np.array([-3.0, 1.0]))
    assert (obs.low, obs.high) == (-2.0, 2.0)
    s, z = obs.scale_and_zero_point(8, "asymmetric")
    assert np.isclose(s, 4.0 / 255) and z == np.round(0 - (-2.0) / s)
    x = np.array([-1.0, -0.5, 0.0, 0.5, 1.0])
    m = oracle.ste_mask(x, 0.5 / 127, 0.0, 8, "symmetric")
    assert m.tolist() == [False, True, True, True, False]


# ---------------------------------------------------------------------------
# GELU: the tanh form of nn/activations.py:32, pinned at non-trivial points
# against a 50-digit evaluation of the same formula, and shown to differ from
# the erf form 0.5 x (1 + erf(x / sqrt 2)) there (x = 0 and large x cannot
# tell the two apart).
# ---------------------------------------------------------------------------
_PI_50 = "3.14159265358979323846264338327950288419716939937510"


def _gelu_tanh_decimal(x: float):
    from decimal import Decimal, getcontext
    getcontext().prec = 50
    d = Decimal(x)
    u = (Decimal(2) / Decimal(_PI_50)).sqrt() * (d + Decimal("0.044715") * d ** 3)
    e2 = (2 * u).exp()
    return Decimal("0.5") * d * (1 + (e2 - 1) / (e2 + 1))


@pytest.mark.parametrize("x", [-3.0, -1.0, -0.5, 0.5, 1.0, 2.0, 3.0])
def test_gelu_is_the_tanh_form(x):
    import math
    want = float(_gelu_tanh_decimal(x))
    got = float(oracle.activate("gelu", np.array([x]))[0])
    assert abs(got - want) <= 4e-16 * max(1.0, abs(want))
    erf_form = 0.5 * x * (1 + math.erf(x / math.sqrt(2)))
    assert abs(erf_form - want) > 1e-5
    # a dropped cubic term moves the value by more than the bound as well
    no_cubic = 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * x))
    assert abs(no_cubic - want) > 1e-5


# ---------------------------------------------------------------------------
# quantization_error (compression/quantization.py:218-229): closed forms.
# ---------------------------------------------------------------------------
def test_quantization_error_closed_forms():
    import math
    # one tensor: diff (1, -2), |a| = 5: relative = sqrt(5) / 5
    r = oracle.quantization_error([np.array([3.0, 4.0])], [np.array([4.0, 2.0])])
    assert r["mean_abs_error"] == 1.5
    assert r["max_abs_error"] == 2.0
    assert r["relative_error"] == pytest.approx(math.sqrt(5) / 5, rel=1e-15)
    # a missing square root in the numerator (1.0) or the denominator
    # (sqrt 5 / 25) would both miss this value
    assert abs(r["relative_error"] - 1.0) > 0.1 and abs(r["relative_error"] - math.sqrt(5) / 25) > 0.1
    # several outputs of different shapes are flattened and concatenated:
    # a = (3, 4, 0, 12), b = (4, 2, 0, 12) -> diff (1, -2, 0, 0), |a| = 13
    r = oracle.quantization_error([np.array([[3.0]]), np.array([4.0, 0.0]), np.array([[12.0]])],
                                  [np.array([[4.0]]), np.array([2.0, 0.0]), np.array([[12.0]])])
    assert r["mean_abs_error"] == 0.75
    assert r["max_abs_error"] == 2.0
    assert r["relative_error"] == pytest.approx(math.sqrt(5) / 13, rel=1e-15)
    # a zero reference gives relative error 0 (the reference's denom > 0 branch)
    r = oracle.quantization_error([np.zeros(3)], [np.array([1.0, -1.0, 2.0])])
    assert r["relative_error"] == 0.0 and r["max_abs_error"] == 2.0
    assert r["mean_abs_error"] == pytest.approx(4.0 / 3.0, rel=1e-15)


# ---------------------------------------------------------------------------
# forward (nn/forward.py:272-811): the layer loop, written out by hand.
# outputs[0] is the input and layer i's output is outputs[i + 1] (:304,
# :810); residual_add adds outputs[save_index] (:762-766); a layer's
# act_quant fake-quantizes its output after the activation (:798-805).
# ---------------------------------------------------------------------------
def _chain_layers(rng):
    def dense(n_in, n_out, act):
        return {"type": "dense", "activation": act,
                "weights": rng.standard_normal((n_out, n_in)) * 0.4,
                "bias": rng.standard_normal(n_out) * 0.1}
    spec = {"bits": 8, "scheme": "asymmetric", "scale": np.array(0.0123),
            "zero_point": np.array(37.0)}
    layers = [dense(6, 8, "relu"),                          # 0 -> outputs[1]
              dense(8, 8, "tanh"),                          # 1 -> outputs[2]
              {"type": "residual_add", "save_index": 1},    # 2 -> outputs[3]
              {"type": "residual_save"},                    # 3 -> outputs[4]
              {"type": "layernorm", "gamma": rng.standard_normal(8),
               "beta": rng.standard_normal(8), "epsilon": 1e-5},   # 4
              dense(8, 8, "linear"),                        # 5
              {"type": "residual_add", "save_index": 4},    # 6: outputs[4]
              dense(8, 5, "sigmoid")]                       # 7
    layers[5]["act_quant"] = spec
    layers[6]["act_quant"] = dict(spec, scale=np.array(0.05), zero_point=np.array(100.0))
    return layers


def _explicit_chain(layers, x, save_shift=0, skip_act_quant=False):
    def fq(v, spec):
        s, zp = float(spec["scale"]), float(spec["zero_point"])
        q = np.clip(np.round(v / s + zp), 0, 255)
        return (q - zp) * s

    def sig(v):
        return 1.0 / (1.0 + np.exp(-v))
    W = [layer.get("weights") for layer in layers]
    B = [layer.get("bias") for layer in layers]
    o = [x]
    o.append(np.maximum(0.0, x @ W[0].T + B[0]))
    o.append(np.tanh(o[1] @ W[1].T + B[1]))
    o.append(o[2] + o[1 + save_shift])
    o.append(o[3])
    g, b = layers[4]["gamma"], layers[4]["beta"]
    mu = o[4].mean(axis=-1, keepdims=True)
    var = ((o[4] - mu) ** 2).mean(axis=-1, keepdims=True)
    o.append(g * (o[4] - mu) / np.sqrt(var + 1e-5) + b)
    z5 = o[5] @ W[5].T + B[5]
    o.append(z5 if skip_act_quant else fq(z5, layers[5]["act_quant"]))
    r = o[6] + o[4 + save_shift]
    o.append(r if skip_act_quant else fq(r, layers[6]["act_quant"]))
    o.append(sig(o[7] @ W[7].T + B[7]))
    return o


def test_forward_matches_explicit_chain():
    rng = np.random.default_rng(41)
    layers = _chain_layers(rng)
    x = rng.standard_normal((5, 6))
    got = oracle.forward(layers, x, dtype=np.float64)
    want = _explicit_chain(layers, x)
    assert len(got) == len(layers) + 1 and got[0] is not None
    for i, (g, w) in enumerate(zip(got, want)):
        assert g.shape == w.shape, i
        assert np.max(np.abs(g - w)) <= 1e-12, f"outputs[{i}]"
    # the act_quant outputs sit on their grids
    for i, li in ((6, 5), (7, 6)):
        spec = layers[li]["act_quant"]
        q = got[i] / float(spec["scale"]) + float(spec["zero_point"])
        assert np.max(np.abs(q - np.round(q))) < 1e-9
    # planted mistakes, each of which the comparison above would catch: a
    # save_index read one output later, act_quant left out, and (below)
    # act_quant applied before a non-linear activation instead of after it
    for kw in ({"save_shift": 1}, {"skip_act_quant": True}):
        bad = _explicit_chain(layers, x, **kw)
        assert max(np.max(np.abs(g - w)) for g, w in zip(got, bad)) > 1e-3, kw
    tl = _chain_layers(np.random.default_rng(41))
    tl[5]["activation"] = "tanh"
    got_t = oracle.forward(tl, x, dtype=np.float64)
    z = got_t[5] @ tl[5]["weights"].T + tl[5]["bias"]
    spec = tl[5]["act_quant"]
    s, zp = float(spec["scale"]), float(spec["zero_point"])
    after = (np.clip(np.round(np.tanh(z) / s + zp), 0, 255) - zp) * s
    before = np.tanh((np.clip(np.round(z / s + zp), 0, 255) - zp) * s)
    assert np.max(np.abs(got_t[6] - after)) <= 1e-12
    assert np.max(np.abs(got_t[6] - before)) > 1e-3


# ---------------------------------------------------------------------------
# Calibration ranges (compression/quantization.py:176-209).  The percentile
# path is NumPy's np.percentile (default 'linear' method): pinned against the
# exact rational interpolation between the two order statistics around
# (n - 1) q / 100, and closed forms on integer ramps.
# ---------------------------------------------------------------------------
def _exact_percentile(values, q):
    # the virtual index as the method defines it on floats, (n - 1) * (q / 100)
    # in float64; the interpolation between the order statistics exact
    s = sorted(Fraction(float(v)) for v in values)
    h = Fraction((len(s) - 1) * (q / 100.0))
    lo = int(h)
    if lo >= len(s) - 1:
        return s[-1]
    return s[lo] + (h - lo) * (s[lo + 1] - s[lo])


@pytest.mark.parametrize("n", [1, 2, 5, 17, 1000])
def test_percentile_is_linear_interpolation(n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n)
    for q in (0.0, 0.1, 12.5, 50.0, 99.0, 99.9, 100.0):
        got = oracle.percentile(x, q)
        want = _exact_percentile(x, q)
        ulp = np.spacing(max(abs(float(want)), 1e-300))
        assert abs(Fraction(got) - want) <= 4 * Fraction(float(ulp)), (n, q)
    # an integer ramp: the percentile is the index itself
    ramp = np.arange(101, dtype=np.float64)
    for q in (0, 1, 37, 50, 99, 100):
        assert oracle.percentile(ramp, q) == q
    assert np.isnan(oracle.percentile(np.array([1.0, np.nan, 3.0]), 50))


def test_observe_ranges_and_specs():
    rng = np.random.default_rng(2)
    outs = [rng.standard_normal((8, 3)), rng.standard_normal((8, 4)) * 3,
            np.arange(6, dtype=np.int64), rng.uniform(0, 1, (8, 2))]
    r = oracle.observe_ranges(outs)
    assert sorted(r) == [0, 2]          # the integer output is skipped
    assert r[0] == [float(outs[1].min()), float(outs[1].max())]
    r = oracle.observe_ranges(outs, percentile_p=90.0)
    assert r[0] == [float(np.percentile(outs[1], 10.0)), float(np.percentile(outs[1], 90.0))]
    # a second batch widens the ranges
    wider = [o * 2 if o.dtype.kind == "f" else o for o in outs]
    r2 = oracle.observe_ranges(wider, percentile_p=90.0, ranges={k: list(v) for k, v in r.items()})
    for k in r:
        assert r2[k][0] == min(r[k][0], 2 * r[k][0]) and r2[k][1] == max(r[k][1], 2 * r[k][1])
    specs = oracle.specs_from_ranges(r)
    low, high = r[2]
    assert float(specs[2]["scale"]) == float(np.float64(high - low) / 255)
    with pytest.raises(RuntimeError):
        oracle.specs_from_ranges({})


def test_w8a8_static_accumulator_and_grid_identity():
    # static W8A8 (calibrated per-tensor activation spec): the accumulator is
    # the exact integer dot product of (q - zp) and the weight codes, and for
    # activations already on the spec's grid, acc * scale * w_scale is the
    # float Dense of the fake-quantized values
    rng = np.random.default_rng(17)
    x = rng.standard_normal((7, 33)).astype(np.float32) * 2
    low, high = float(x.min()), float(x.max())
    scale, zp = oracle.compute_scale(np.asarray(low), np.asarray(high), 8, "asymmetric")
    spec = {"bits": 8, "scheme": "asymmetric", "scale": scale, "zero_point": zp}
    assert float(zp) != 0.0
    x_fq = oracle.fake_quantize(x, scale, zp, 8, "asymmetric").astype(np.float32)
    w = (rng.standard_normal((5, 33)) * 0.1).astype(np.float32)
    w_codes, w_scale = oracle.int8_codes(w, per_channel=True)
    y, acc, q = oracle.w8a8_static_dense(x_fq, spec, w_codes, w_scale.reshape(-1))
    zi = int(zp)
    exact = [[sum((int(q[i, k]) - zi) * int(w_codes[j, k]) for k in range(33)) for j in range(5)]
             for i in range(7)]
    assert np.array_equal(acc, np.array(exact, np.int32))
    fq_w = w_codes.astype(np.float64) * w_scale.astype(np.float64).reshape(-1, 1)
    # the grid values themselves, (q - zp) * scale in float64
    grid = (q.astype(np.float64) - float(zp)) * float(scale)
    want = grid @ fq_w.T
    got = acc * float(scale) * w_scale.astype(np.float64).reshape(1, -1)
    assert np.max(np.abs(got - want)) <= 1e-12 * np.abs(want).max()
    # the float32 fake-quantized activations differ from the grid by their rounding
    want32 = x_fq.astype(np.float64) @ fq_w.T
    assert np.max(np.abs(y - want32)) <= 1e-5 * np.abs(want32).max()
    # planted mistake: the zero point left out of the accumulator
    bad = np.dot(q.astype(np.float64), w_codes.astype(np.float64).T)
    assert not np.array_equal(bad.astype(np.int64), acc.astype(np.int64))
