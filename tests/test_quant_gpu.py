"""GPU parity of the quantization kernels with the NumPy oracle.

Bar: bit-identical outputs (values, signed zeros, dtypes, shapes); NaN
positions must agree (NaN payloads are not compared)."""

import copy

import numpy as np
import pytest

import enilnets_amd as ea
from enilnets_amd.nn.dense import quantize_rows_i8
from enilnets_amd.device import DeviceArray
import oracle

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    """Bit-identical arrays (dtype and shape included), any NaN for NaN."""
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == b.dtype, (a.dtype, b.dtype)
    assert a.shape == b.shape, (a.shape, b.shape)
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb), "NaN positions differ"
    ua = a[~na].view(np.uint64 if a.dtype == np.float64 else np.uint32)
    ub = b[~nb].view(np.uint64 if b.dtype == np.float64 else np.uint32)
    bad = np.nonzero(ua != ub)[0]
    assert bad.size == 0, f"{bad.size} elements differ, first: {a[~na][bad[:5]]} vs {b[~nb][bad[:5]]}"


def check_tensor(w, **kw):
    got = ea.quantize_tensor(w, **kw)
    want = oracle.quantize_tensor(w, **kw)
    for g, o in zip(got, want):
        assert type(g) is type(o)
        same_bits(g, o)


SHAPES = [(1,), (3,), (7, 13), (512, 512), (1000003,), (64, 1000), (10, 1024), (1024, 784),
          (33, 4099), (3, 40000), (5, 70000)]


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("per_channel", [False, True])
def test_quantize_tensor_symmetric(gpu, dtype, shape, per_channel):
    rng = np.random.default_rng(abs(hash((shape, per_channel))) % 2**32)
    w = (rng.standard_normal(shape) * rng.uniform(0.01, 3.0)).astype(dtype)
    check_tensor(w, bits=8, per_channel=per_channel)


@pytest.mark.parametrize("bits", [2, 4, 8, 12, 16])
@pytest.mark.parametrize("scheme", ["symmetric", "asymmetric"])
@pytest.mark.parametrize("per_channel", [False, True])
def test_quantize_tensor_bits_schemes(gpu, bits, scheme, per_channel):
    rng = np.random.default_rng(bits * 7 + per_channel)
    w = rng.uniform(-0.7, 2.3, (37, 129)).astype(np.float32)
    check_tensor(w, bits=bits, scheme=scheme, per_channel=per_channel)


@pytest.mark.parametrize("axis", [0, 1, 2, -1, 5])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_quantize_tensor_axes(gpu, axis, dtype):
    rng = np.random.default_rng(100 + axis)
    w = rng.standard_normal((6, 7, 50)).astype(dtype)
    check_tensor(w, bits=8, per_channel=True, axis=axis)
    check_tensor(w, bits=6, scheme="asymmetric", per_channel=True, axis=axis)


def test_quantize_tensor_stacked_experts(gpu):
    # MoE layout (E, H, D): per_channel=True gives one scale per expert
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((8, 256, 1024)) * 0.02).astype(np.float32)
    check_tensor(w, bits=8, per_channel=True)


def test_special_values(gpu):
    w = np.array([[0.0, -0.0, 1e-45, -3e-44, 2.5, -2.5],
                  [np.nan, 1.0, -1.0, 0.0, 0.0, 0.0],
                  [np.inf, 1.0, 2.0, -1.0, 0.5, 0.0],
                  [-np.inf, 3.0, 0.0, 0.0, 0.0, 0.0],
                  [0.0, 0.0, 0.0, 0.0, 0.0, -0.0],
                  [3e38, -3e38, 1.0, 1e-30, -1e-30, 7.0],
                  [1e-40, -1e-41, 1e-42, 0.0, -1e-40, 5e-41]], np.float32)
    for per_channel in (False, True):
        for scheme in ("symmetric", "asymmetric"):
            check_tensor(w, bits=8, scheme=scheme, per_channel=per_channel)
    check_tensor(w.astype(np.float64), bits=8, per_channel=True)


def test_integer_input_promotes_to_float64(gpu):
    w = np.arange(-50, 70).reshape(10, 12)
    check_tensor(w, bits=8, per_channel=True)
    check_tensor(w, bits=4, scheme="asymmetric")


def test_empty_raises(gpu):
    with pytest.raises(ValueError):
        ea.quantize_tensor(np.zeros((0, 3), np.float32))


BCAST = [(), (4, 1, 1), (1, 5, 1), (1, 1, 6), (6,), (4, 5, 1), (4, 1, 6), (1, 5, 6), (4, 5, 6)]


@pytest.mark.parametrize("sshape", BCAST)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_quantize_dequantize_fake_broadcast(gpu, sshape, dtype):
    rng = np.random.default_rng(len(sshape) * 11 + sum(sshape))
    x = rng.standard_normal((4, 5, 6)).astype(dtype)
    scale = rng.uniform(0.01, 0.2, sshape).astype(dtype)
    zp = np.round(rng.uniform(0, 10, sshape)).astype(dtype)
    for scheme, z in (("symmetric", np.zeros_like(scale)), ("asymmetric", zp)):
        same_bits(ea.quantize(x, scale, z, 8, scheme), oracle.quantize(x, scale, z, 8, scheme))
        same_bits(ea.fake_quantize(x, scale, z, 6, scheme),
                  oracle.fake_quantize(x, scale, z, 6, scheme))
        codes = oracle.quantize(x, scale, z, 8, scheme)
        same_bits(ea.dequantize(codes, scale, z), oracle.dequantize(codes, scale, z))


def test_mixed_types_promote_like_numpy(gpu):
    x = np.linspace(-1, 1, 11).astype(np.float32)
    for scale, zp in ((0.01, 0.0), (np.float64(0.01), 0.0), (np.array(0.01), np.float32(0)),
                      (np.float32(0.01), 0)):
        got = ea.quantize(x, scale, zp, 8, "symmetric")
        want = oracle.quantize(x, scale, zp, 8, "symmetric")
        assert type(got) is type(want)
        same_bits(got, want)
    # scalar input gives a scalar, like NumPy
    got = ea.quantize(np.float32(0.3), np.float32(0.01), np.float32(0), 8, "symmetric")
    want = oracle.quantize(np.float32(0.3), np.float32(0.01), np.float32(0), 8, "symmetric")
    assert type(got) is type(want) and got == want
    ints = np.arange(-5, 5)
    same_bits(ea.dequantize(ints, np.float32(0.5), 0), oracle.dequantize(ints, np.float32(0.5), 0))


@pytest.mark.parametrize("scheme", ["symmetric", "asymmetric"])
def test_compute_scale(gpu, scheme):
    rng = np.random.default_rng(3)
    low = -np.abs(rng.standard_normal((9, 1))).astype(np.float32)
    high = np.abs(rng.standard_normal((9, 1))).astype(np.float32)
    low[0] = 0
    high[0] = 0
    low[1] = np.nan
    for bits in (3, 8, 16):
        for g, o in zip(ea.compute_scale(low, high, bits, scheme),
                        oracle.compute_scale(low, high, bits, scheme)):
            assert type(g) is type(o)
            same_bits(g, o)
    for g, o in zip(ea.compute_scale(-1.5, 2.0, 8, scheme), oracle.compute_scale(-1.5, 2.0, 8,
                                                                                   scheme)):
        assert type(g) is type(o)
        same_bits(g, o)


def _model(rng):
    class M:
        pass
    m = M()
    m.layers = [
        {"type": "dense", "weights": (rng.standard_normal((64, 48)) * 0.1).astype(np.float32),
         "bias": np.zeros(64, np.float32), "activation": "relu", "use_bias": True,
         "activation_params": {}},
        {"type": "residual_save"},
        {"type": "moe", "W1": (rng.standard_normal((4, 16, 64)) * 0.1).astype(np.float32),
         "W2": (rng.standard_normal((4, 64, 16)) * 0.1).astype(np.float32),
         "Wr": (rng.standard_normal((4, 64)) * 0.1).astype(np.float32)},
        {"type": "dense", "weights": (rng.standard_normal((10, 64)) * 0.1).astype(np.float32),
         "bias": np.zeros(10, np.float32), "activation": "linear", "use_bias": True,
         "activation_params": {}},
    ]
    return m


@pytest.mark.parametrize("per_channel", [False, True])
@pytest.mark.parametrize("bits,scheme", [(8, "symmetric"), (4, "asymmetric")])
def test_quantize_weights(gpu, per_channel, bits, scheme):
    rng = np.random.default_rng(9)
    m = _model(rng)
    a, b = copy.deepcopy(m), copy.deepcopy(m)
    ra = ea.quantize_weights(a, bits=bits, scheme=scheme, per_channel=per_channel)
    rb = oracle.quantize_weights(b, bits=bits, scheme=scheme, per_channel=per_channel)
    for la, lb in zip(a.layers, b.layers):
        for name in oracle.QUANTIZABLE.get(la["type"], ()):
            same_bits(la[name], lb[name])
            for key in ("scale", "zero_point"):
                same_bits(la["quant"][name][key], lb["quant"][name][key])
            assert la["quant"][name]["bits"] == bits and la["quant"][name]["scheme"] == scheme
    assert set(ra) == set(rb)
    for key in ("bits", "scheme", "per_channel", "parameters", "float_bytes",
                "quantized_bytes", "compression"):
        assert ra[key] == rb[key]
    assert ra["mean_abs_error"] == pytest.approx(rb["mean_abs_error"], rel=1e-5)
    assert ra["layers"].keys() == rb["layers"].keys()
    for k in ra["layers"]:
        assert ra["layers"][k]["size"] == rb["layers"][k]["size"]
        assert ra["layers"][k]["mean_abs_error"] == pytest.approx(
            rb["layers"][k]["mean_abs_error"], rel=1e-5)
    # layer_types filter
    c = copy.deepcopy(m)
    rc = ea.quantize_weights(c, layer_types=["moe"])
    assert list(rc["layers"]) == ["2.W1", "2.W2", "2.Wr"]
    assert "quant" not in c.layers[0]


def test_quantization_error(gpu):
    rng = np.random.default_rng(10)
    ref = [rng.standard_normal((30, 7)).astype(np.float32), rng.standard_normal(5).astype(np.float32)]
    cand = [r + rng.standard_normal(r.shape).astype(np.float32) * 1e-3 for r in ref]
    got = ea.quantization_error(ref, cand)
    want = oracle.quantization_error(ref, cand)
    for k in want:
        assert got[k] == pytest.approx(want[k], rel=1e-5)
    assert ea.quantization_error(ref, ref)["max_abs_error"] == 0.0


@pytest.mark.parametrize("shape", [(1, 1), (16, 8192), (4096, 1024), (300, 784), (7, 100003),
                                   (5, 33)])
def test_int8_rows(gpu, shape):
    rng = np.random.default_rng(shape[0])
    x = (rng.standard_normal(shape) * 2).astype(np.float32)
    x[0, 0] = -0.0
    codes, scale = quantize_rows_i8(DeviceArray.from_numpy(x))
    want_codes, want_scale = oracle.int8_codes(x, per_channel=True)
    assert np.array_equal(codes.numpy(), want_codes)
    same_bits(scale.numpy(), want_scale.reshape(-1))


# (outer, channels, inner) layouts of enq_dequantize_i8: per-channel rows,
# per-tensor (one channel), a middle channel axis; shapes with n % 4 == 0 and
# inner % 4 == 0 take dequant_i8_kernel, the rest the elementwise kernel
DEQUANT_LAYOUTS = [(1, 33, 70), (1, 64, 1024), (1, 8192, 256), (1, 1, 65536), (1, 1, 1003),
                   (3, 5, 64), (2, 7, 9), (1, 8192, 8192)]


@pytest.mark.parametrize("outer,channels,inner", DEQUANT_LAYOUTS)
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_dequantize_i8(gpu, outer, channels, inner, dtype):
    from enilnets_amd import _lib
    if outer * channels * inner > 1 << 24 and dtype == np.float64:
        pytest.skip("the float32 case covers the full-size layout")
    print(f"[case] dequantize_i8 {outer}x{channels}x{inner} {np.dtype(dtype).name}", flush=True)
    rng = np.random.default_rng(channels + inner)
    codes = rng.integers(-127, 128, (outer, channels, inner), dtype=np.int8)
    scale = (rng.uniform(0.5, 2.0, (1, channels, 1)) * 0.01).astype(dtype)
    d_c, d_s = DeviceArray.from_numpy(codes), DeviceArray.from_numpy(scale.reshape(-1))
    out = DeviceArray(codes.shape, dtype)
    code = _lib.F32 if dtype == np.float32 else _lib.F64
    _lib.call("enq_dequantize_i8", code, d_c.ptr, outer, channels, inner, d_s.ptr, out.ptr)
    want = oracle.dequantize(codes.astype(dtype), scale, np.zeros_like(scale))
    assert want.dtype == dtype
    assert np.array_equal(out.numpy(), want)   # == semantics: int8 0 gives +0.0


def test_dequantize_i8_unaligned_output(gpu):
    # an output that is not 16-byte aligned takes the elementwise kernel on
    # purpose; the values are the same
    import ctypes
    from enilnets_amd import _lib
    rng = np.random.default_rng(13)
    codes = rng.integers(-127, 128, (64, 1024), dtype=np.int8)
    scale = (rng.uniform(0.5, 2.0, 64) * 0.01).astype(np.float32)
    d_c, d_s = DeviceArray.from_numpy(codes), DeviceArray.from_numpy(scale)
    buf = DeviceArray.from_numpy(np.zeros(codes.size + 4, np.float32))
    _lib.call("enq_dequantize_i8", _lib.F32, d_c.ptr, 1, 64, 1024, d_s.ptr,
              ctypes.c_void_p(buf.address + 4))
    got = buf.numpy()
    want = oracle.dequantize(codes.astype(np.float32), scale.reshape(-1, 1), np.float32(0))
    assert np.array_equal(got[1:1 + codes.size].reshape(codes.shape), want)
    assert got[0] == 0 and not got[1 + codes.size:].any()


def test_quantize_tensor_per_channel_8192(gpu):
    # BASELINE configs[2]'s weight through the public API (row kernel) and
    # its int8 codes, bit-exact; the codes dequantize back to the fake floats
    from enilnets_amd import _lib
    from enilnets_amd.nn.dense import quantize_weight_rows
    print("[case] quantize_tensor per channel 8192x8192", flush=True)
    rng = np.random.default_rng(8192)
    w = rng.normal(0.0, 0.02, (8192, 8192)).astype(np.float32)
    got = ea.quantize_tensor(w, 8, "symmetric", per_channel=True)
    want = oracle.quantize_tensor(w, 8, "symmetric", per_channel=True)
    assert np.array_equal(got[0], want[0])
    same_bits(got[1], want[1])
    same_bits(got[2], want[2])
    rows = quantize_weight_rows(w)
    want_codes, want_scale = oracle.int8_codes(w, per_channel=True)
    assert np.array_equal(rows.codes.numpy(), want_codes)
    same_bits(rows.scale.numpy(), want_scale.reshape(-1))
    out = DeviceArray(w.shape, np.float32)
    _lib.call("enq_dequantize_i8", _lib.F32, rows.codes.ptr, 1, 8192, 8192, rows.scale.ptr,
              out.ptr)
    assert np.array_equal(out.numpy(), want[0])


@pytest.mark.parametrize("shape", [(64, 48), (1024, 784), (10, 1024), (300, 2000), (33, 9000)])
@pytest.mark.parametrize("per_channel", [False, True])
def test_quantize_weights_keeps_device_int8_codes(gpu, shape, per_channel):
    # the codes cached for the integer kernels equal the oracle's codes
    from enilnets_amd.nn.weights import int8_weights
    rng = np.random.default_rng(shape[0])

    class M:
        pass
    m = M()
    w = (rng.standard_normal(shape) * 0.05).astype(np.float32)
    m.layers = [{"type": "dense", "weights": w, "bias": np.zeros(shape[0], np.float32),
                 "activation": "linear"}]
    ea.quantize_weights(m, bits=8, per_channel=per_channel)
    wq = int8_weights(m.layers[0], "weights")
    want_codes, want_scale = oracle.int8_codes(w, per_channel=per_channel)
    assert np.array_equal(wq.codes.numpy(), want_codes)
    rows = np.broadcast_to(np.asarray(want_scale, np.float32).reshape(-1), (shape[0],)) \
        if per_channel else np.full(shape[0], np.float32(want_scale))
    assert np.array_equal(wq.scale.numpy(), rows)


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_codes_at_unaligned_offsets(gpu, offset):
    # int8 codes written at any byte offset: the vector kernels store four
    # codes as one 32-bit word, so they may only take a 4-byte aligned output
    import ctypes
    from enilnets_amd import _lib
    rng = np.random.default_rng(offset)
    n = 4099 * 3
    w = (rng.standard_normal(n) * 0.05).astype(np.float32)
    want_codes, want_scale = oracle.int8_codes(w, per_channel=False)
    d_w = DeviceArray.from_numpy(w)
    scale, zp = DeviceArray((1,), np.float32), DeviceArray((1,), np.float32)
    for entry in ("enq_quantize_tensor", "enq_quantize_codes_i8"):
        buf = DeviceArray.from_numpy(np.zeros(n + 8, np.int8))
        dst = ctypes.c_void_p(buf.address + offset)
        if entry == "enq_quantize_tensor":
            _lib.call(entry, _lib.F32, d_w.ptr, 1, 1, n, 8, _lib.SYMMETRIC, None, dst,
                      scale.ptr, zp.ptr, None)
            same_bits(scale.numpy(), np.asarray(want_scale, np.float32).reshape(-1))
        else:
            _lib.call(entry, _lib.F32, d_w.ptr, 1, 1, n, scale.ptr, zp.ptr, -127, 127, dst)
        got = buf.numpy()
        assert np.array_equal(got[offset:offset + n], want_codes.reshape(-1)), entry
        assert not got[:offset].any() and not got[offset + n:].any(), entry


# per-tensor float32 tensors of whole 8192-value rows: the range reduction,
# then one row kernel with the shared scale; every output combination
PER_TENSOR_ROWS = [((2, 8192), 8, "symmetric", False), ((16, 8192), 4, "asymmetric", False),
                   ((96, 1024), 7, "asymmetric", True), ((8192, 8192), 8, "symmetric", False)]


@pytest.mark.parametrize("shape,bits,scheme,special", PER_TENSOR_ROWS)
def test_quantize_per_tensor_whole_rows(gpu, shape, bits, scheme, special):
    from enilnets_amd import _lib
    print(f"[case] per-tensor rows {shape} {bits} {scheme} special={special}", flush=True)
    rng = np.random.default_rng(shape[0] * 31 + bits)
    w = (rng.standard_normal(shape) * 0.05).astype(np.float32)
    if special:
        w.reshape(-1)[[5, 700, 9000]] = [np.inf, -0.0, 1e-42]
    want_fake, want_scale, want_zp = oracle.quantize_tensor(w, bits, scheme, per_channel=False)
    q = oracle.quantize(w, want_scale, want_zp, bits, scheme)
    want_codes = np.where(np.isnan(q), 0, q).astype(np.int8)
    d_w = DeviceArray.from_numpy(w)
    sch = _lib.SYMMETRIC if scheme == "symmetric" else _lib.ASYMMETRIC
    for want_f, want_c in ((True, True), (False, True), (True, False)):
        fake = DeviceArray(shape, np.float32) if want_f else None
        codes = DeviceArray(shape, np.int8) if want_c else None
        scale, zp = DeviceArray((1,), np.float32), DeviceArray((1,), np.float32)
        _lib.call("enq_quantize_tensor", _lib.F32, d_w.ptr, 1, 1, w.size, bits, sch,
                  fake.ptr if fake else None, codes.ptr if codes else None, scale.ptr, zp.ptr,
                  None)
        same_bits(scale.numpy(), np.asarray(want_scale, np.float32).reshape(-1))
        same_bits(zp.numpy(), np.asarray(want_zp, np.float32).reshape(-1))
        if fake:
            same_bits(fake.numpy(), want_fake)
        if codes:
            assert np.array_equal(codes.numpy(), want_codes)
