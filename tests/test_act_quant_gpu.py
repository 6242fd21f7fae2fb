"""GPU parity of activation fake-quantization (``act_quant``,
``Enilnets/nn/forward.py:798-805``; specs from ``ActivationCalibrator``,
``compression/quantization.py:156-209``).

* The standalone pass is bit-identical to the oracle's ``fake_quantize`` in
  the arithmetic NumPy picks (float64 for the calibrator's float64 scale,
  float32 for float32 specs), rounded to float32.
* The Dense epilogue that fuses it is bit-identical to the unfused Dense
  followed by the standalone pass, on the GEMV and both GEMM tile paths and
  after a softmax.
* ``Forward`` with calibrated specs matches the oracle's ``forward``: the
  layer GEMMs are not bit-exact, so an output may land on the neighbouring
  grid point (about 2 x 1e-5 x 255 = 0.5% of outputs for an 8-bit grid);
  every element is within one quantization step and fewer than 2% differ
  beyond float32 rounding.
"""

import numpy as np
import pytest

import enilnets_amd as ea
from enilnets_amd.device import DeviceArray
from enilnets_amd.nn import Model
from enilnets_amd.nn import dense as D
from enilnets_amd.nn.weights import Int8Weights
import oracle

pytestmark = pytest.mark.gpu


def spec_for(x, bits=8, scheme="asymmetric", dtype=np.float64):
    low, high = float(np.min(x)), float(np.max(x))
    scale, zp = oracle.compute_scale(np.asarray(low, dtype), np.asarray(high, dtype), bits, scheme)
    return {"bits": bits, "scheme": scheme, "scale": scale, "zero_point": zp}


@pytest.mark.parametrize("dtype,scheme,bits", [(np.float64, "asymmetric", 8),
                                               (np.float32, "asymmetric", 8),
                                               (np.float64, "symmetric", 8),
                                               (np.float64, "asymmetric", 4)])
def test_standalone_pass_bit_exact(gpu, dtype, scheme, bits):
    rng = np.random.default_rng(bits)
    x = (rng.standard_normal(100003) * 3).astype(np.float32)
    x[:5] = [0.0, -0.0, np.nan, 1e30, -1e30]
    spec = spec_for(x[5:], bits, scheme, dtype)
    want = oracle.fake_quantize(x, spec["scale"], spec["zero_point"], bits, scheme)
    assert want.dtype == np.result_type(np.float32, dtype)
    got = D.act_quant(DeviceArray.from_numpy(x), spec).numpy()
    w32 = want.astype(np.float32)
    nan = np.isnan(w32)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), w32[~nan].view(np.uint32))


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 4096 * 1024 + 2])
@pytest.mark.parametrize("in_place", [False, True])
def test_standalone_pass_sizes(gpu, n, in_place):
    # the vector kernel (16-byte aligned, n >= 4) with its n % 4 tail, and
    # the scalar kernel below 4 values; in place as Forward applies it
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 2).astype(np.float32)
    for spec_dtype in (np.float64, np.float32):
        spec = spec_for(x if n > 1 else np.array([-1.0, 1.0]), 8, "asymmetric", spec_dtype)
        want = oracle.fake_quantize(x, spec["scale"], spec["zero_point"], 8,
                                    "asymmetric").astype(np.float32)
        d_x = DeviceArray.from_numpy(x)
        got = D.act_quant(d_x, spec, out=d_x if in_place else None).numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("scale", [0.1, 0.02, 1.0 / 3.0, 0.0234375, 3.7, 1e-3])
@pytest.mark.parametrize("zp", [0.0, 3.0, 117.0])
def test_standalone_pass_rounding_ties(gpu, scale, zp):
    """Quotients x / scale + zp on and next to half-integers.  With the scale
    rounded to 15 significant bits every (k + 0.5 - zp) * scale is a float32,
    so those quotients are exact ties (rounded half to even); their float32
    neighbours sit just off the tie.  The float64 path multiplies by the
    reciprocal and must hand exact ties to the true division."""
    e = np.floor(np.log2(scale))
    s15 = float(np.round(scale / 2.0 ** (e - 14)) * 2.0 ** (e - 14))
    k = np.arange(-140, 141, dtype=np.float64)
    ties = ((k + 0.5 - zp) * s15).astype(np.float32)
    assert np.array_equal(ties.astype(np.float64) / s15 + zp, k + 0.5)
    up1 = np.nextafter(ties, np.float32(np.inf))
    dn1 = np.nextafter(ties, np.float32(-np.inf))
    up2 = np.nextafter(up1, np.float32(np.inf))
    rng = np.random.default_rng(int(scale * 1e4) + int(zp))
    noise = (rng.standard_normal(4096) * 140 * s15).astype(np.float32)
    x = np.concatenate([ties, up1, dn1, up2, noise])
    spec = {"bits": 8, "scheme": "asymmetric", "scale": np.float64(s15),
            "zero_point": np.float64(zp)}
    want = oracle.fake_quantize(x, spec["scale"], spec["zero_point"], 8, "asymmetric")
    assert want.dtype == np.float64
    got = D.act_quant(DeviceArray.from_numpy(x), spec).numpy()
    w32 = want.astype(np.float32)
    assert np.array_equal(got.view(np.uint32), w32.view(np.uint32))


def make_w(rng, n, k):
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    fq, scale, _ = oracle.quantize_tensor(w, 8, per_channel=True)
    codes = oracle.quantize(w, scale, np.zeros_like(scale), 8, "symmetric").astype(np.int8)
    rows = np.ascontiguousarray(scale.reshape(-1).astype(np.float32))
    return Int8Weights(DeviceArray.from_numpy(codes), DeviceArray.from_numpy(rows), codes.shape,
                       8, True, None, None)


@pytest.mark.parametrize("m,k,n,act", [(8, 512, 300, "relu"), (4096, 1024, 10, "linear"),
                                       (300, 784, 1024, "gelu"), (2048, 1024, 4096, "relu"),
                                       (100, 64, 37, "softmax"), (65, 96, 130, "sigmoid")])
def test_fused_epilogue_equals_separate_pass(gpu, m, k, n, act):
    print(f"[case] dense_w8_aq m={m} k={k} n={n} act={act}", flush=True)
    rng = np.random.default_rng(m + n)
    w = make_w(rng, n, k)
    x = DeviceArray.from_numpy(rng.standard_normal((m, k)).astype(np.float32))
    b = DeviceArray.from_numpy((rng.standard_normal(n) * 0.1).astype(np.float32))
    plain = D.dense_w8(x, w, b, act)
    spec = spec_for(plain.numpy())
    out_dtype = np.float64 if act == "gelu" else np.float32
    fused = D.dense_w8(x, w, b, act, act_quant=spec, out_dtype=out_dtype).numpy()
    separate = D.act_quant(plain, spec, out_dtype).numpy()
    assert np.array_equal(fused.view(np.uint32), separate.view(np.uint32))


def test_forward_with_calibrated_activations(gpu):
    rng = np.random.default_rng(31)
    m = Model()
    m.add_dense((rng.standard_normal((256, 100)) * 0.1).astype(np.float32),
                (rng.standard_normal(256) * 0.01).astype(np.float32), "relu")
    m.add_dense((rng.standard_normal((128, 256)) * 0.1).astype(np.float32),
                (rng.standard_normal(128) * 0.01).astype(np.float32), "gelu")
    m.add_dense((rng.standard_normal((10, 128)) * 0.1).astype(np.float32),
                (rng.standard_normal(10) * 0.01).astype(np.float32), "linear")
    ea.quantize_weights(m, per_channel=True)
    x = rng.uniform(0, 1, (512, 100)).astype(np.float32)
    cal = ea.ActivationCalibrator(m)
    cal.observe(x)
    installed = cal.apply()
    assert sorted(installed) == [0, 1, 2]
    m.Forward(x)
    want = oracle.forward(m.layers, x, dtype=np.float32)
    for i in range(1, 4):
        g, w_ = m.outputs[i], want[i]
        assert g.dtype == w_.dtype, (i, g.dtype, w_.dtype)
        step = float(m.layers[i - 1]["act_quant"]["scale"])
        diff = np.abs(g.astype(np.float64) - w_.astype(np.float64))
        assert np.all(diff <= 1.0001 * step), f"layer {i}: {diff.max()} > {step}"
        # a pre-quantization value within the GEMM's ~1e-5 relative error of a
        # rounding boundary may round the other way: about 2 * 1e-5 * 255
        # grid steps = 0.5% of outputs, a little more after a flipped input
        off = diff > 1e-6 * np.max(np.abs(w_))
        assert off.mean() < 2e-2, f"layer {i}: {off.mean():.2e} of outputs off the oracle's grid point"
    ea.remove_activation_quantization(m)
    assert all("act_quant" not in L for L in m.layers)


# ---------------------------------------------------------------------------
# Percentile calibration (quantization.py:183-188): the device order
# statistics with NumPy's 'linear' interpolation give np.percentile's value
# bit for bit (== semantics: -0.0 and +0.0 are equal, as NumPy's sort
# treats them).
# ---------------------------------------------------------------------------
def _percentile_cases():
    rng = np.random.default_rng(5)
    ties = rng.integers(-3, 4, 5000).astype(np.float32)
    zeros = np.array([0.0, -0.0, 1.0, -0.0, 0.0, -1.0], np.float32)
    inf = rng.standard_normal(300).astype(np.float32)
    inf[[3, 70]] = [np.inf, -np.inf]
    nan = rng.standard_normal(100).astype(np.float32)
    nan[17] = np.nan
    return [("one", np.array([2.5], np.float32)), ("two", np.array([1.0, -4.0], np.float64)),
            ("normal", rng.standard_normal((64, 1000)).astype(np.float32)),
            ("normal64", rng.standard_normal(70001)), ("ties", ties), ("zeros", zeros),
            ("inf", inf), ("nan", nan),
            ("relu", np.maximum(rng.standard_normal(1 << 20), 0).astype(np.float32)),
            # past 2^24 elements the float32 virtual index rounds, as NumPy's does
            ("big", rng.standard_normal((1 << 24) + 5).astype(np.float32))]


@pytest.mark.parametrize("case", range(10))
def test_percentile_matches_numpy(gpu, case):
    from enilnets_amd.compression.quantization import _percentiles
    name, x = _percentile_cases()[case]
    print(f"[case] percentile {name} n={x.size}", flush=True)
    qs = (0.0, 0.1, 1.0, 37.5, 50.0, 99.0, 99.9, 100.0)
    got = _percentiles(x, qs)
    for q, g in zip(qs, got):
        want = oracle.percentile(x, q)
        assert (np.isnan(g) and np.isnan(want)) or g == want, (name, q, g, want)


def test_percentile_calibration(gpu):
    # ActivationCalibrator(percentile=p) over two batches: ranges and specs
    # identical to the reference's observe / apply on the same layer outputs
    rng = np.random.default_rng(44)
    m = Model()
    m.add_dense((rng.standard_normal((256, 100)) * 0.1).astype(np.float32),
                (rng.standard_normal(256) * 0.01).astype(np.float32), "relu")
    m.add_dense((rng.standard_normal((64, 256)) * 0.1).astype(np.float32),
                (rng.standard_normal(64) * 0.01).astype(np.float32), "gelu")
    ea.quantize_weights(m, per_channel=True)
    for p in (99.9, 95.0):
        cal = ea.ActivationCalibrator(m, percentile=p)
        ranges = {}
        for seed in (1, 2):
            x = np.random.default_rng(seed).uniform(0, 1, (300, 100)).astype(np.float32)
            cal.observe(x)
            ranges = oracle.observe_ranges(m.outputs, percentile_p=p, ranges=ranges)
        assert cal.ranges == ranges
        installed = cal.apply()
        want = oracle.specs_from_ranges(ranges)
        for i in want:
            for key in ("scale", "zero_point", "low", "high"):
                assert np.array_equal(installed[i][key], want[i][key]), (p, i, key)
        # a clipped range lies inside the full one over the same batches
        ea.remove_activation_quantization(m)
        full = ea.ActivationCalibrator(m)
        for seed in (1, 2):
            full.observe(np.random.default_rng(seed).uniform(0, 1, (300, 100)).astype(np.float32))
        for i in ranges:
            assert full.ranges[i][0] <= ranges[i][0] <= ranges[i][1] <= full.ranges[i][1]
    with pytest.raises(ValueError):
        ea.ActivationCalibrator(m, percentile=101.0).observe(x)
