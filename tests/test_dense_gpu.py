"""GPU parity of the Dense kernels on int8 weights.

* W8 fp32 variant: max |z - z_ref| <= 1e-4 * max |z_ref| per row, where z_ref
  is the float64 product of the activations with the fake-quantized weights
  (the reference's Dense, ``nn/forward.py:318-319``).
* W8 bf16 variant: the same bound at 2e-2.
* A single output column (n = 1) is bounded against sum_k |x_k w_k| instead of
  |z|, since the row bound there fails for any float32 dot product.
* W8A8: int32 accumulators, activation codes and scales bit-identical to the
  oracle; the linear fp32 output too (same operation order, no FMA).
"""

import numpy as np
import pytest

from enilnets_amd.device import DeviceArray
from enilnets_amd.nn import dense as D
from enilnets_amd.nn.weights import Int8Weights
import oracle

pytestmark = pytest.mark.gpu


def make(m, k, n, seed, per_channel=True, wstd=0.05):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * wstd).astype(np.float32)
    b = (rng.standard_normal(n) * 0.01).astype(np.float32)
    fq, scale, _ = oracle.quantize_tensor(w, 8, per_channel=per_channel)
    codes = oracle.quantize(w, scale, np.zeros_like(scale), 8, "symmetric").astype(np.int8)
    rows = np.broadcast_to(np.asarray(scale, np.float32).reshape(-1, 1)[:, 0]
                           if np.ndim(scale) else np.full(n, scale, np.float32), (n,))
    wq = Int8Weights(DeviceArray.from_numpy(codes), DeviceArray.from_numpy(np.ascontiguousarray(rows)),
                     codes.shape, 8, per_channel, None, None)
    return x, fq, codes, np.ascontiguousarray(rows), b, wq


def row_rel_err(got, ref):
    denom = np.maximum(np.max(np.abs(ref), axis=-1), 1e-30)
    return np.max(np.abs(got - ref), axis=-1) / denom


SHAPES = [(1, 512, 512), (3, 100, 10), (16, 8192, 1024), (16, 784, 1024), (17, 1024, 300),
          (33, 512, 100), (64, 512, 512), (65, 784, 1024), (100, 100, 37), (256, 1024, 1024),
          (300, 784, 1024), (512, 4096, 1024), (1000, 1024, 10), (4, 16, 1), (129, 48, 260),
          # tall-skinny outputs (GEMV over 16-row blocks): ragged K, n = 1, n = 32
          (4096, 1024, 10), (2000, 100, 1), (70, 30, 32), (77, 130, 17)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("variant,tol", [("fp32", 1e-4), ("bf16", 2e-2)])
def test_dense_w8_pre_activation(gpu, m, k, n, variant, tol):
    print(f"[case] dense_w8 {variant} m={m} k={k} n={n}", flush=True)
    x, fq, codes, rows, b, wq = make(m, k, n, seed=m * 31 + k + n)
    z_ref = x.astype(np.float64) @ fq.astype(np.float64).T + b
    d_x, d_b = DeviceArray.from_numpy(x), DeviceArray.from_numpy(b)
    z = DeviceArray((m, n), np.float32)
    y = D.dense_w8(d_x, wq, d_b, "linear", variant=variant, pre_activation=z)
    zh, yh = z.numpy(), y.numpy()
    assert np.array_equal(zh, yh)
    if n == 1:
        # One output per row: the row bound becomes a relative bound on a
        # single dot product, which no float32 evaluation meets under
        # cancellation (the reference's own float32 x @ W misses it on 2 of
        # these 2000 rows).  Bound the error by the magnitude of the terms
        # instead: |z - z_ref| <= tol * sum_k |x_k * w_k|.
        terms = np.abs(x.astype(np.float64)) @ np.abs(fq.astype(np.float64)).T
        err = (np.abs(zh.astype(np.float64) - z_ref) / np.maximum(terms, 1e-30)).max(axis=-1)
    else:
        err = row_rel_err(zh.astype(np.float64), z_ref)
    assert np.all(err <= tol), f"max row error {err.max():.3e} > {tol}"


def test_dense_w8_large_gemv_and_gemm(gpu):
    # BASELINE config 3 shapes; rows of the GEMM checked on a sample
    for m in (16, 4096):
        print(f"[case] dense_w8 fp32 m={m} k=8192 n=8192", flush=True)
        x, fq, codes, rows, b, wq = make(m, 8192, 8192, seed=m, wstd=0.02)
        y = D.dense_w8(DeviceArray.from_numpy(x), wq, None, "linear").numpy()
        pick = np.random.default_rng(0).choice(m, size=min(m, 48), replace=False)
        ref = x[pick].astype(np.float64) @ fq.astype(np.float64).T
        assert np.all(row_rel_err(y[pick].astype(np.float64), ref) <= 1e-4)


# 256 x 256 tiles (at least as many tiles as CUs): the kernel reads the fp32
# activations and splits them itself; partial row and column tiles, a K tail
# (K % 32 == 16), and activations at an address that is not 16-byte aligned
# (the bf16 planes are then split in a separate pass)
BIG_SHAPES = [(4096, 1024, 4096, 0), (4100, 1040, 4100, 0), (4097, 2048, 4095, 4),
              (4096, 512, 4096, 4)]


@pytest.mark.parametrize("m,k,n,offset", BIG_SHAPES)
@pytest.mark.parametrize("variant,tol", [("fp32", 1e-4), ("bf16", 2e-2)])
def test_dense_w8_big_tiles(gpu, m, k, n, offset, variant, tol):
    print(f"[case] dense_w8 big {variant} m={m} k={k} n={n} offset={offset}", flush=True)
    x, fq, codes, rows, b, wq = make(m, k, n, seed=m + k + n + offset, wstd=0.03)
    if offset:
        # the same activations one float past a 16-byte boundary
        buf = DeviceArray.from_numpy(np.concatenate([np.zeros(offset // 4, np.float32),
                                                     x.reshape(-1)]))
        d_x = DeviceArray((m, k), np.float32, ptr=buf.address + offset, owner=buf)
    else:
        d_x = DeviceArray.from_numpy(x)
    z = DeviceArray((m, n), np.float32)
    y = D.dense_w8(d_x, wq, DeviceArray.from_numpy(b), "relu", variant=variant,
                   pre_activation=z)
    zh, yh = z.numpy(), y.numpy()
    pick = np.unique(np.concatenate([np.arange(0, m, 37), np.arange(m - 5, m)]))
    z_ref = x[pick].astype(np.float64) @ fq.astype(np.float64).T + b
    err = row_rel_err(zh[pick].astype(np.float64), z_ref)
    assert np.all(err <= tol), f"max row error {err.max():.3e} > {tol}"
    assert np.array_equal(yh, np.maximum(zh, 0))


@pytest.mark.parametrize("m,k,n", [(4096, 1024, 4096), (300, 784, 1024), (4100, 1040, 4100),
                                   (129, 100, 37), (65, 48, 260)])
@pytest.mark.parametrize("variant,tol", [("fp32", 1e-4), ("bf16", 2e-2)])
def test_dense_w8_on_split_planes(gpu, m, k, n, variant, tol):
    # split once, multiply twice: within the Dense bound, and for the large
    # tiles (where dense_w8 itself splits in a separate pass) bit-identical
    # to dense_w8
    print(f"[case] dense_w8_planes {variant} m={m} k={k} n={n}", flush=True)
    x, fq, codes, rows, b, wq = make(m, k, n, seed=m + 2 * k + n, wstd=0.03)
    d_x, d_b = DeviceArray.from_numpy(x), DeviceArray.from_numpy(b)
    xp = D.split_planes(d_x, variant)
    for act in ("linear", "gelu"):
        z = DeviceArray((m, n), np.float32)
        y = D.dense_w8_planes(xp, wq, d_b, act, pre_activation=z).numpy()
        zh = z.numpy()
        pick = np.unique(np.concatenate([np.arange(0, m, 41), [m - 1]]))
        z_ref = x[pick].astype(np.float64) @ fq.astype(np.float64).T + b
        assert np.all(row_rel_err(zh[pick].astype(np.float64), z_ref) <= tol)
        assert np.allclose(y, oracle.activate(act, zh.astype(np.float64)), rtol=2e-6, atol=2e-6)
        if variant == "bf16" and (m + 255) // 256 * ((n + 255) // 256) >= 256:
            # (the large fp32 tiles of dense_w8 take the fp16 / e4m3 split,
            # compared with dense_w8_split below)
            y2 = D.dense_w8(d_x, wq, d_b, act, variant=variant).numpy()
            assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


def e4m3_round(v):
    """Nearest OCP e4m3 value (bias 7, 3 mantissa bits, subnormals down to
    2^-9), ties to even; |v| stays below the format's 448 here."""
    v = np.asarray(v, np.float64)
    a = np.abs(v)
    ex = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    ulp = np.exp2(np.maximum(ex, -6.0) - 3.0)
    return np.sign(v) * np.round(a / ulp) * ulp


def e4m3_value(b):
    b = np.asarray(b, np.uint8).astype(np.int64)
    s, e, f = b >> 7, (b >> 3) & 15, b & 7
    mag = np.where(e == 0, np.ldexp(f / 8.0, -6), np.ldexp(1.0 + f / 8.0, e - 7))
    return np.where(s == 1, -mag, mag)


def wide_rows(m, k, seed):
    """Activation rows of very different kinds: normal, a zero row, rows
    scaled by 1e-30 and 1e30, heavy-tailed (Cauchy), log-normal magnitudes,
    a row with a few outliers a thousand times the rest."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k))
    kinds = np.arange(m) % 7
    x[kinds == 1] = 0.0
    x[kinds == 2] *= 1e-30
    x[kinds == 3] *= 1e30
    x[kinds == 4] = rng.standard_cauchy((int(np.sum(kinds == 4)), k))
    x[kinds == 5] *= np.exp(rng.normal(0.0, 3.0, (int(np.sum(kinds == 5)), k)))
    x[kinds == 6, : min(k, 8)] *= 1000.0
    return x.astype(np.float32)


@pytest.mark.parametrize("m,k", [(9, 8192), (7, 100), (7, 1040), (7, 9000)])
def test_split_f16f8_layout(gpu, m, k):
    # the split of the large-tile fp32 path, element by element: the row
    # exponent, hi = fp16(x * 2^e) and lo = e4m3(x * 2^e - hi), zero padding
    print(f"[case] split_f16f8 m={m} k={k}", flush=True)
    x = wide_rows(m, k, seed=m + k)
    buf = D.split_f16f8(DeviceArray.from_numpy(x)).data.numpy()
    kp = -(-k // 64) * 64
    hi = buf[: 2 * m * kp].view(np.uint16).reshape(m, kp)
    lo = buf[2 * m * kp: 3 * m * kp].reshape(m, kp)
    ex = buf[3 * m * kp:].view(np.int32)
    amax = np.max(np.abs(x), axis=1)
    want_e = np.where(amax > 0, 15 - np.frexp(np.where(amax > 0, amax, 1.0))[1], 0)
    assert np.array_equal(ex, want_e)
    xs = np.ldexp(x, want_e[:, None]).astype(np.float32)
    h = xs.astype(np.float16)
    assert np.array_equal(hi[:, :k], h.view(np.uint16))
    r = (xs - h.astype(np.float32)).astype(np.float64)
    assert np.array_equal(e4m3_value(lo[:, :k]), e4m3_round(r))
    assert not hi[:, k:].any() and not lo[:, k:].any()


@pytest.mark.parametrize("m,k,n", [(4096, 1024, 4096), (4100, 1040, 4100), (4097, 2048, 4095),
                                   (4096, 1024, 3072), (1024, 2304, 4096), (300, 784, 1024),
                                   (129, 48, 260), (65, 64, 32)])
def test_dense_w8_split(gpu, m, k, n):
    # the fp16 / e4m3 split GEMM within the fp32 bound on rows of every kind,
    # and, where dense_w8 takes it (tiles that fill the device, or more than
    # 2^33 multiply-adds), bit-identical to dense_w8
    print(f"[case] dense_w8_split m={m} k={k} n={n}", flush=True)
    _, fq, codes, rows, b, wq = make(m, k, n, seed=3 * m + k + n, wstd=0.03)
    x = wide_rows(m, k, seed=m + n)
    d_x, d_b = DeviceArray.from_numpy(x), DeviceArray.from_numpy(b)
    xs = D.split_f16f8(d_x)
    z = DeviceArray((m, n), np.float32)
    y = D.dense_w8_split(xs, wq, d_b, "relu", pre_activation=z).numpy()
    zh = z.numpy()
    pick = np.unique(np.concatenate([np.arange(0, m, 29), np.arange(m - 8, m)]))
    z_ref = x[pick].astype(np.float64) @ fq.astype(np.float64).T + b
    err = row_rel_err(zh[pick].astype(np.float64), z_ref)
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e}"
    assert np.array_equal(y, np.maximum(zh, 0))
    if (m + 255) // 256 * ((n + 255) // 256) >= 256 or m * n * k > 2 ** 33:
        y2 = D.dense_w8(d_x, wq, d_b, "relu").numpy()
        assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("act", ["relu", "leakyrelu", "elu", "selu", "gelu", "swish", "mish",
                                 "sigmoid", "tanh", "softplus", "softmax"])
def test_dense_w8_activations(gpu, act):
    print(f"[case] activation {act}", flush=True)
    x, fq, codes, rows, b, wq = make(96, 256, 130, seed=7)
    z = DeviceArray((96, 130), np.float32)
    y = D.dense_w8(DeviceArray.from_numpy(x), wq, DeviceArray.from_numpy(b), act,
                   pre_activation=z).numpy()
    zh = z.numpy()
    want = oracle.activate(act, zh.astype(np.float64))
    assert np.allclose(y, want, rtol=2e-6, atol=2e-6)


@pytest.mark.parametrize("m,k,n", [(3, 100, 10), (40, 128, 300), (77, 130, 17), (4096, 1024, 10)])
@pytest.mark.parametrize("act", ["relu", "gelu", "elu", "softmax"])
def test_dense_w8_gemv_direct_activations(gpu, m, k, n, act):
    # GEMV shapes with a single K slice: the decode (m <= 64) and skinny
    # (n <= 32) kernels apply the scale, bias and activation themselves
    print(f"[case] gemv direct {act} m={m} k={k} n={n}", flush=True)
    x, fq, codes, rows, b, wq = make(m, k, n, seed=m + 3 * k + n)
    z = DeviceArray((m, n), np.float32)
    y = D.dense_w8(DeviceArray.from_numpy(x), wq, DeviceArray.from_numpy(b), act,
                   pre_activation=z).numpy()
    zh = z.numpy()
    z_ref = x.astype(np.float64) @ fq.astype(np.float64).T + b
    assert np.all(row_rel_err(zh.astype(np.float64), z_ref) <= 1e-4)
    want = oracle.activate(act, zh.astype(np.float64))
    assert np.allclose(y, want, rtol=2e-6, atol=2e-6)


def test_dense_w8_rejects_bad_shapes(gpu):
    x, fq, codes, rows, b, wq = make(4, 32, 8, seed=1)
    with pytest.raises(ValueError):
        D.dense_w8(DeviceArray.from_numpy(np.zeros((4, 31), np.float32)), wq)
    with pytest.raises(ValueError):
        D.dense_w8(DeviceArray.from_numpy(x), wq, activation="bogus")


W8A8_SHAPES = [(1, 64, 64), (7, 100, 33), (16, 8192, 512), (64, 784, 1024), (200, 1000, 300),
               (256, 1024, 1024), (512, 4096, 1024), (1000, 48, 10), (130, 16, 70),
               (4096, 1024, 4096),
               # 256 x 256 ring kernel (>= 128 tiles): a single K stage, a K
               # shorter than the ring, and a K tail with partial row and
               # column tiles
               (4096, 16, 2048), (4096, 208, 2048), (4000, 1040, 2100)]


@pytest.mark.parametrize("m,k,n", W8A8_SHAPES)
def test_w8a8_bit_exact(gpu, m, k, n):
    print(f"[case] w8a8 m={m} k={k} n={n}", flush=True)
    x, fq, codes, rows, b, wq = make(m, k, n, seed=m + k * 3 + n)
    y_ref, acc_ref, xs_ref, xc_ref = oracle.w8a8_dense(x, codes, rows, b)
    d_x = DeviceArray.from_numpy(x)
    xc, xs = D.quantize_rows_i8(d_x)
    assert np.array_equal(xc.numpy(), xc_ref)
    assert np.array_equal(xs.numpy(), xs_ref.reshape(-1))
    acc = DeviceArray((m, n), np.int32)
    y = D.dense_w8a8(d_x, wq, DeviceArray.from_numpy(b), "linear", acc=acc)
    assert np.array_equal(acc.numpy(), acc_ref)
    assert np.array_equal(y.numpy(), y_ref)
    acc2 = DeviceArray((m, n), np.int32)
    y2 = D.gemm_w8a8(xc, xs, wq, DeviceArray.from_numpy(b), acc=acc2)
    assert np.array_equal(acc2.numpy(), acc_ref)
    assert np.array_equal(y2.numpy(), y_ref)


def test_w8a8_square_8192(gpu):
    print("[case] w8a8 8192^3", flush=True)
    rng = np.random.default_rng(77)
    xc = rng.integers(-127, 128, (8192, 8192), dtype=np.int8)
    wc = rng.integers(-127, 128, (8192, 8192), dtype=np.int8)
    xs = np.full(8192, 0.01, np.float32)
    ws = np.full(8192, 0.02, np.float32)
    wq = Int8Weights(DeviceArray.from_numpy(wc), DeviceArray.from_numpy(ws), wc.shape, 8, True,
                     None, None)
    acc = DeviceArray((8192, 8192), np.int32)
    D.gemm_w8a8(DeviceArray.from_numpy(xc), DeviceArray.from_numpy(xs), wq, acc=acc)
    got = acc.numpy()
    pick = rng.choice(8192, size=24, replace=False)
    want = (xc[pick].astype(np.float64) @ wc.astype(np.float64).T).astype(np.int64)
    assert np.array_equal(got[pick].astype(np.int64), want)
    # a checksum of all rows: sum over n of acc equals x . (sum of W rows)
    wsum = wc.astype(np.int64).sum(axis=0)
    assert np.array_equal(got.astype(np.int64).sum(axis=1), xc.astype(np.int64) @ wsum)


STATIC_SPECS = [("asymmetric", 8, np.float64), ("symmetric", 8, np.float32),
                ("asymmetric", 4, np.float64), ("symmetric", 8, np.float64)]


@pytest.mark.parametrize("m,k,n", [(64, 512, 300), (4096, 1024, 4096), (300, 1000, 70),
                                   (200, 1040, 2100)])
@pytest.mark.parametrize("spec_i", range(len(STATIC_SPECS)))
def test_w8a8_static(gpu, m, k, n, spec_i):
    # activations quantized with a calibrated per-tensor spec: int32
    # accumulators and the linear output bit-identical to the composed
    # oracle; on activations the spec already fake-quantized, within the
    # Dense bound of the reference's float Dense of those values
    scheme, bits, sdt = STATIC_SPECS[spec_i]
    print(f"[case] w8a8 static {scheme}{bits} {np.dtype(sdt).name} m={m} k={k} n={n}", flush=True)
    x, fq, codes, rows, b, wq = make(m, k, n, seed=m + k + n + spec_i)
    x = x * 1.5 + 0.25
    low, high = float(x.min()), float(x.max())
    scale, zp = oracle.compute_scale(np.asarray(low, sdt), np.asarray(high, sdt), bits, scheme)
    spec = {"bits": bits, "scheme": scheme, "scale": scale, "zero_point": zp}
    x_fq = oracle.fake_quantize(x, scale, zp, bits, scheme).astype(np.float32)
    for xin in (x_fq, x):
        acc = DeviceArray((m, n), np.int32)
        y = D.dense_w8a8(DeviceArray.from_numpy(xin), wq, DeviceArray.from_numpy(b), "linear",
                         acc=acc, x_spec=spec).numpy()
        y_ref, acc_ref, _ = oracle.w8a8_static_dense(xin, spec, codes, rows, b)
        assert np.array_equal(acc.numpy(), acc_ref)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    z_ref = x_fq.astype(np.float64) @ fq.astype(np.float64).T + b
    y = D.dense_w8a8(DeviceArray.from_numpy(x_fq), wq, DeviceArray.from_numpy(b), "relu",
                     x_spec=spec).numpy()
    err = np.max(np.abs(y - np.maximum(z_ref, 0)), axis=1) / np.max(np.abs(z_ref), axis=1)
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e}"


# (m, k, n1, n2, act1, bias): the configs[3] feed-forward pair (fused: the
# first GEMM writes the second's fp16/e4m3 split), a ReLU pair with biases
# (fused), and a small pair through two Dense calls
FFN_CASES = [(4096, 1024, 4096, 1024, "gelu", False), (4096, 512, 8192, 1024, "relu", True),
             (300, 96, 200, 50, "gelu", True)]


@pytest.mark.parametrize("m,k,n1,n2,act1,bias", FFN_CASES)
def test_dense_w8_ffn(gpu, m, k, n1, n2, act1, bias):
    print(f"[case] dense_w8_ffn m={m} k={k} n1={n1} n2={n2} {act1} bias={bias}", flush=True)
    x, fq1, _, _, bb1, wq1 = make(m, k, n1, seed=m + k + n1, wstd=0.02)
    _, fq2, _, _, bb2, wq2 = make(8, n1, n2, seed=n1 + n2, wstd=0.02)
    if not bias:
        bb1, bb2 = np.zeros_like(bb1), np.zeros_like(bb2)
    d_x = DeviceArray.from_numpy(x)
    d_b1, d_b2 = DeviceArray.from_numpy(bb1), DeviceArray.from_numpy(bb2)
    y = D.dense_w8_ffn(d_x, wq1, d_b1, act1, wq2, d_b2, "linear").numpy()
    # rows checked against float64 on a sample of at most 64
    pick = np.unique(np.linspace(0, m - 1, min(m, 64)).astype(np.int64))
    h = oracle.activate(act1, x[pick].astype(np.float64) @ fq1.astype(np.float64).T + bb1)
    ref = h @ fq2.astype(np.float64).T + bb2
    err = row_rel_err(y[pick].astype(np.float64), ref)
    assert np.all(err <= 1e-4), f"max row error {err.max():.3e}"
    assert np.isfinite(y).all()
    # the same as two dense_w8 calls, to the same bar
    h2 = D.dense_w8(d_x, wq1, d_b1, act1)
    y2 = D.dense_w8(h2, wq2, d_b2, "linear").numpy()
    assert np.all(row_rel_err(y2[pick].astype(np.float64), ref) <= 1e-4)
    assert np.all(row_rel_err(y.astype(np.float64), y2.astype(np.float64)) <= 2e-4)
    # a bound computed once per weight gives the same output, bit for bit
    bound = D.ffn_bound(wq1, d_b1, act1)
    y3 = D.dense_w8_ffn(d_x, wq1, d_b1, act1, wq2, d_b2, "linear", bound=bound).numpy()
    assert np.array_equal(y3, y)


def test_dense_w8_ffn_bf16_and_errors(gpu):
    # the bf16 variant takes two Dense calls (bf16 bar, 2e-2 of the row)
    x, fq1, _, _, bb1, wq1 = make(512, 256, 512, seed=5, wstd=0.02)
    _, fq2, _, _, bb2, wq2 = make(8, 512, 128, seed=6, wstd=0.02)
    d_x = DeviceArray.from_numpy(x)
    d_b1, d_b2 = DeviceArray.from_numpy(bb1), DeviceArray.from_numpy(bb2)
    y = D.dense_w8_ffn(d_x, wq1, d_b1, "gelu", wq2, d_b2, "linear", variant="bf16").numpy()
    h = oracle.activate("gelu", x.astype(np.float64) @ fq1.astype(np.float64).T + bb1)
    ref = h @ fq2.astype(np.float64).T + bb2
    assert np.all(row_rel_err(y.astype(np.float64), ref) <= 2e-2)
    # misaligned shapes, and an output bound for softmax (which has none)
    with pytest.raises(ValueError):
        D.dense_w8_ffn(d_x, wq1, d_b1, "gelu", wq1, d_b2, "linear")
    with pytest.raises(ValueError):
        D.ffn_bound(wq1, d_b1, "softmax")
