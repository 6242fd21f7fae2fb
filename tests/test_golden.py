"""Golden fixtures (tests/golden/, written by make_fixtures.py from the oracle).

CPU tests: the oracle still reproduces the committed vectors (a regression
pin for the checker).  GPU tests: the HIP path reproduces them (bit-exact for
codes, scales and accumulators; fp32 tolerance for Dense outputs)."""

import os
import sys

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)

import make_fixtures as mf  # noqa: E402
import oracle  # noqa: E402


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def codes_digest(codes):
    c = codes.astype(np.int64)
    return int(c.sum()), int((c * np.arange(c.size).reshape(c.shape)).sum())


def test_oracle_reproduces_config0():
    g = load("config0_dense.npz")
    w, b, x = mf.config0()
    fq, scale, _ = oracle.quantize_tensor(w, 8)
    codes = oracle.quantize(w, scale, np.zeros_like(scale), 8, "symmetric").astype(np.int8)
    assert np.array_equal(scale, g["scale"]) and scale.dtype == g["scale"].dtype
    assert np.array_equal(codes[:64], g["codes_head"])
    assert codes_digest(codes) == (int(g["codes_checksum"]), int(g["codes_weighted"]))
    y, _ = oracle.dense_forward({"weights": fq, "bias": b, "activation": "linear"},
                                x.astype(np.float64), np.float64)
    assert np.array_equal(y[:16], g["y_head"])


def test_oracle_reproduces_per_channel():
    g = load("per_channel.npz")
    w = mf.per_channel_case()
    assert np.array_equal(w, g["w"], equal_nan=True)
    fq, scale, zp = oracle.quantize_tensor(w, 8, per_channel=True)
    for a, key in ((fq, "fake"), (scale, "scale"), (zp, "zp")):
        assert np.array_equal(a, g[key], equal_nan=True)
    fqa, sa, za = oracle.quantize_tensor(w, 6, "asymmetric", per_channel=True)
    for a, key in ((fqa, "fake_asym6"), (sa, "scale_asym6"), (za, "zp_asym6")):
        assert np.array_equal(a, g[key], equal_nan=True)


def test_oracle_reproduces_w8a8():
    g = load("w8a8.npz")
    x, w, b = mf.w8a8_case()
    codes, s = oracle.int8_codes(w, per_channel=True)
    y, acc, xs, xc = oracle.w8a8_dense(x, codes, s.reshape(-1), b)
    for a, key in ((codes, "w_codes"), (s, "w_scale"), (xc, "x_codes"), (xs, "x_scale"),
                   (acc, "acc"), (y, "y")):
        assert np.array_equal(a, g[key])


def test_oracle_reproduces_moe():
    g = load("moe.npz")
    layer, x, logits = mf.moe_case()
    e = np.exp(logits - logits.max(axis=1, keepdims=True))
    probs = e / e.sum(axis=1, keepdims=True)
    assert np.array_equal(oracle.forward_top_k(probs, 2), g["top"])
    l64 = {k: (v.astype(np.float64) if isinstance(v, np.ndarray) else v) for k, v in layer.items()}
    y = oracle.moe_forward(x.astype(np.float64), l64, probs.astype(np.float64))
    assert np.allclose(y, g["y"], rtol=0, atol=1e-12)


@pytest.mark.gpu
def test_gpu_config0(gpu):
    import enilnets_amd as ea
    from enilnets_amd.nn import int8_weights
    g = load("config0_dense.npz")
    w, b, x = mf.config0()
    fq, scale, zp = ea.quantize_tensor(w, 8)
    assert np.array_equal(scale, g["scale"]) and scale.dtype == g["scale"].dtype
    model = ea.Model()
    model.add_dense(w, b, "linear")
    ea.quantize_weights(model, bits=8)
    codes = int8_weights(model.layers[0], "weights").codes.numpy()
    assert np.array_equal(codes[:64], g["codes_head"])
    assert codes_digest(codes) == (int(g["codes_checksum"]), int(g["codes_weighted"]))
    y = model.Forward(x)
    ref = g["y_head"]
    err = np.max(np.abs(y[:16] - ref), axis=1) / np.max(np.abs(ref), axis=1)
    assert np.all(err <= 1e-4)


@pytest.mark.gpu
def test_gpu_per_channel(gpu):
    import enilnets_amd as ea
    g = load("per_channel.npz")
    w = g["w"]
    for args, keys in ((dict(bits=8, per_channel=True), ("fake", "scale", "zp")),
                       (dict(bits=6, scheme="asymmetric", per_channel=True),
                        ("fake_asym6", "scale_asym6", "zp_asym6"))):
        got = ea.quantize_tensor(w, **args)
        for a, key in zip(got, keys):
            assert a.dtype == g[key].dtype and a.shape == g[key].shape
            assert np.array_equal(a, g[key], equal_nan=True)


@pytest.mark.gpu
def test_gpu_w8a8(gpu):
    from enilnets_amd.device import DeviceArray
    from enilnets_amd.nn import dense as D
    from enilnets_amd.nn.weights import Int8Weights
    g = load("w8a8.npz")
    x, w, b = mf.w8a8_case()
    wq = Int8Weights(DeviceArray.from_numpy(g["w_codes"]),
                     DeviceArray.from_numpy(g["w_scale"].reshape(-1)), g["w_codes"].shape, 8,
                     True, None, None)
    acc = DeviceArray(g["acc"].shape, np.int32)
    y = D.dense_w8a8(DeviceArray.from_numpy(x), wq, DeviceArray.from_numpy(b), acc=acc)
    assert np.array_equal(acc.numpy(), g["acc"])
    assert np.array_equal(y.numpy(), g["y"])
