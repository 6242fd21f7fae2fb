"""Host-side logic of the drop-in API (no GPU): validation, dtype and shape
resolution, broadcasting layout, layer-dict handling."""

import copy

import numpy as np
import pytest

import enilnets_amd as ea
from enilnets_amd.compression import quantization as q
from enilnets_amd.nn import weights as wmod
import oracle


def test_quant_range_matches_reference_contract():
    for bits in range(2, 17):
        for scheme in ("symmetric", "asymmetric"):
            assert ea.quant_range(bits, scheme) == oracle.quant_range(bits, scheme)
    for bad in ((1, "symmetric"), (17, "symmetric"), (8, "bogus"), (0, "asymmetric")):
        with pytest.raises(ValueError):
            ea.quant_range(*bad)


def test_validation_precedes_device_use():
    # invalid bits/scheme raise ValueError before any device call
    for fn, args in ((ea.quantize, ([1.0], 1.0, 0.0, 1, "symmetric")),
                     (ea.fake_quantize, ([1.0], 1.0, 0.0, 8, "nope")),
                     (ea.compute_scale, (0.0, 1.0, 20, "symmetric")),
                     (ea.quantize_tensor, ([1.0, 2.0], 99))):
        with pytest.raises(ValueError):
            fn(*args)


@pytest.mark.parametrize("out_shape,params,expect", [
    ((4, 5, 6), [np.ones(()), np.zeros(())], (1, 1, 120)),
    ((4, 5, 6), [np.ones((4, 1, 1)), np.zeros(())], (1, 4, 30)),
    ((4, 5, 6), [np.ones((1, 5, 1)), np.zeros((5, 1))], (4, 5, 6)),
    ((4, 5, 6), [np.ones((6,)), np.zeros(())], (20, 6, 1)),
    ((4, 5, 6), [np.ones((4, 5, 1)), np.zeros(())], (1, 20, 6)),
    ((4, 5, 6), [np.ones((4, 1, 6)), np.zeros(())], (1, 120, 1)),
    ((8, 1), [np.ones((8, 1)), np.zeros((8, 1))], (1, 8, 1)),
])
def test_channel_layout(out_shape, params, expect):
    outer, channels, inner, flats = q._channel_layout(out_shape, params, np.float32)
    assert (outer, channels, inner) == expect
    for p, f in zip(params, flats):
        assert f.size == channels and f.dtype == np.float32
        # every element's channel value equals the broadcast parameter
        full = np.broadcast_to(np.asarray(p, np.float32), out_shape).reshape(-1)
        idx = np.arange(full.size)
        ch = (idx // inner) % channels
        assert np.array_equal(full, f[ch])


@pytest.mark.parametrize("x,scale", [
    (np.ones(3, np.float32), np.float32(0.5)),
    (np.ones(3, np.float32), 0.5),
    (np.ones(3, np.float32), np.array(0.5)),
    (np.ones(3), np.float32(0.5)),
    (np.ones(3, np.int64), 0.5),
    (np.ones(3, np.float32), np.ones((3,), np.float64)),
])
def test_probe_dtype_matches_numpy(x, scale):
    want = np.clip(np.round(x / scale + 0.0), -127, 127)
    like = np.clip(np.round(q._probe(x) / q._probe(scale) + q._probe(0.0)), -127, 127)
    assert np.result_type(like) == want.dtype


def test_tensor_layout_axis_semantics():
    w = np.zeros((3, 4, 5))
    assert q._tensor_layout(w, True, 0) == (1, 3, 20, (3, 1, 1))
    assert q._tensor_layout(w, True, 1) == (3, 4, 5, (1, 4, 1))
    assert q._tensor_layout(w, True, 2) == (12, 5, 1, (1, 1, 5))
    # an axis that matches no dimension reduces every axis (keepdims)
    assert q._tensor_layout(w, True, -1) == (1, 1, 60, (1, 1, 1))
    assert q._tensor_layout(w, False, 0) == (1, 1, 60, ())
    assert q._tensor_layout(np.zeros(7), True, 0) == (1, 1, 7, ())
    # the oracle agrees on the scale shapes
    for axis in (0, 1, 2, -1):
        s = oracle.quantize_tensor(np.arange(60.0).reshape(3, 4, 5), per_channel=True,
                                   axis=axis)[1]
        assert s.shape == q._tensor_layout(w, True, axis)[3]


def test_unsupported_dtypes_raise():
    with pytest.raises(NotImplementedError):
        q._compute_code(np.float16)
    with pytest.raises(NotImplementedError):
        q._compute_code(np.complex64)


def test_row_scales_expansion():
    assert np.array_equal(wmod._row_scales((3, 4), np.float32(2.0)), [2.0, 2.0, 2.0])
    s = np.arange(3, dtype=np.float32).reshape(3, 1)
    assert np.array_equal(wmod._row_scales((3, 4), s), [0, 1, 2])
    e = np.array([1.0, 2.0], np.float32).reshape(2, 1, 1)
    assert np.array_equal(wmod._row_scales((2, 3, 4), e), [1, 1, 1, 2, 2, 2])


def test_int8_cache_is_dropped_by_deepcopy():
    layer = {"_state_enq_int8": {"weights": wmod.Int8Weights.__new__(wmod.Int8Weights)}}
    clone = copy.deepcopy(layer)
    assert clone["_state_enq_int8"]["weights"] is None


def test_unquantized_dense_is_refused():
    layer = {"type": "dense", "weights": np.ones((2, 2), np.float32), "bias": np.zeros(2)}
    with pytest.raises(NotImplementedError):
        wmod.int8_weights(layer, "weights")


def test_activation_args():
    from enilnets_amd.nn.dense import activation_args
    assert activation_args("relu") == (1, 0.01, 500.0)
    assert activation_args("elu") == (3, 1.0, 500.0)
    assert activation_args("leakyrelu", {"alpha": 0.2})[1] == pytest.approx(0.2)
    with pytest.raises(ValueError):
        activation_args("bogus")


def test_int8_file_round_trips_unquantized_layers(tmp_path):
    # no int8 weights: no device needed; every value, dtype and key order back
    from enilnets_amd.nn import LoadInt8, Model, SaveInt8
    m = Model()
    m.add_dense(np.arange(12, dtype=np.float32).reshape(3, 4), activation="relu")
    m.add_layernorm(3, epsilon=1e-6)
    m.layers[0]["act_quant"] = {"bits": 8, "scheme": "asymmetric", "scale": np.asarray(0.5),
                                "zero_point": np.float64(3.0), "low": -1.0, "high": 2.0}
    m.layers[1]["_state_scratch"] = np.zeros(2)
    f = tmp_path / "model.int8"
    info = SaveInt8(m, str(f))
    assert info == {"int8_bytes": 0, "float_bytes": 0}
    m2 = LoadInt8(str(f))
    assert list(m2.layers[0]) == list(m.layers[0])
    assert "_state_scratch" not in m2.layers[1]
    for a, b in zip(m.layers, m2.layers):
        for k, v in b.items():
            if isinstance(v, np.ndarray):
                assert v.dtype == a[k].dtype and np.array_equal(v, a[k])
    aq = m2.layers[0]["act_quant"]
    assert type(aq["scale"]) is np.ndarray and aq["scale"].dtype == np.float64
    assert type(aq["zero_point"]) is np.float64 and aq["low"] == -1.0


def test_int8_file_rejects_other_archives(tmp_path):
    from enilnets_amd.nn import LoadInt8
    f = tmp_path / "other.npz"
    meta = np.frombuffer(b'{"format": "something-else", "version": 1}', dtype=np.uint8)
    with open(f, "wb") as fh:
        np.savez(fh, meta=meta)
    with pytest.raises(ValueError):
        LoadInt8(str(f))


def test_init_weights_layout_and_methods():
    # nn/weight_init.py:11-46: weights (n_out, n_in) float32, zero bias, the
    # method's bounds; orthogonal rows orthonormal; unknown names raise
    from enilnets_amd.nn.weight_init import init_weights
    np.random.seed(3)
    for method in ("xavier_uniform", "xavier_normal", "he_uniform", "he_normal", "normal",
                   "orthogonal", "zeros", "ones"):
        w, b = init_weights(40, 24, method=method)
        assert w.shape == (24, 40) and w.dtype == np.float32
        assert b.shape == (24,) and not b.any()
    w, _ = init_weights(40, 24, "xavier_uniform")
    assert np.abs(w).max() <= np.sqrt(6 / 64) and np.abs(w).max() > 0.5 * np.sqrt(6 / 64)
    w, _ = init_weights(40, 24, "he_uniform")
    assert np.abs(w).max() <= np.sqrt(6 / 40)
    w, _ = init_weights(40, 24, "orthogonal")
    assert np.allclose(w @ w.T, np.eye(24), atol=1e-5)
    # a seeded run draws the same weights twice
    np.random.seed(11)
    w1, _ = init_weights(7, 5, "he_normal")
    np.random.seed(11)
    w2, _ = init_weights(7, 5, "he_normal")
    assert np.array_equal(w1, w2)
    with pytest.raises(ValueError):
        init_weights(4, 4, "nope")
