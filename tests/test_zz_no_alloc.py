"""The allocation-free Dense entry point (``enq_dense_w8_noalloc``).

It has no counterpart in the reference; it is checked against
``enq_dense_w8``, which runs the same kernels: outputs bit-identical, called
through the C-ABI, twice in a row with the second call smaller (the fixed
scratch keeps the first call's contents), on each path that takes scratch
(decode GEMV partials, skinny GEMV partials, bf16 activation planes) and on
the fused paths that take none; a call needing more than the 64 MiB scratch
fails before launching anything and leaves its output untouched.
"""

import ctypes

import numpy as np
import pytest

from enilnets_amd import _lib
from enilnets_amd.device import DeviceArray
import oracle

pytestmark = pytest.mark.gpu

LINEAR, RELU = 0, 1


def _weights(rng, n, k):
    w = (rng.standard_normal((n, k)) * 0.03).astype(np.float32)
    codes, scale = oracle.int8_codes(w, per_channel=True)
    return (DeviceArray.from_numpy(codes),
            DeviceArray.from_numpy(np.ascontiguousarray(scale.reshape(-1), np.float32)))


def _call(entry, x, m, k, codes, scale, n, bias, act, variant, y, z):
    _lib.call(entry, x.ptr, m, k, codes.ptr, scale.ptr, n, bias.ptr if bias else None, act,
              ctypes.c_float(0.01), ctypes.c_float(500.0), variant, y.ptr, z.ptr if z else None)


def _both(rng, m, k, n, act, variant, weights=None):
    codes, scale = weights or _weights(rng, n, k)
    x = DeviceArray.from_numpy(rng.standard_normal((m, k)).astype(np.float32))
    b = DeviceArray.from_numpy((rng.standard_normal(n) * 0.01).astype(np.float32))
    outs = []
    for entry in ("enq_dense_w8", "enq_dense_w8_noalloc"):
        y, z = DeviceArray((m, n), np.float32), DeviceArray((m, n), np.float32)
        _call(entry, x, m, k, codes, scale, n, b, act, variant, y, z)
        outs.append((y.numpy(), z.numpy()))
    (y0, z0), (y1, z1) = outs
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
    assert np.array_equal(z0.view(np.uint32), z1.view(np.uint32))
    return codes, scale


# (first call, smaller second call): m, k, n, variant
CASES = [
    ("decode gemv", (16, 8192, 8192, _lib.W8_FP32), (5, 8192, 4096, _lib.W8_FP32)),
    ("decode gemv m<=64", (64, 4096, 2048, _lib.W8_FP32), (33, 1024, 1000, _lib.W8_BF16)),
    ("skinny gemv", (4096, 8192, 10, _lib.W8_FP32), (700, 4096, 7, _lib.W8_FP32)),
    ("bf16 planes", (4096, 4096, 8192, _lib.W8_BF16), (4096, 1040, 4100, _lib.W8_BF16)),
    ("fused tiles", (4096, 1024, 4096, _lib.W8_FP32), (300, 784, 1024, _lib.W8_FP32)),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_noalloc_matches_dense_w8(gpu, case):
    name, first, second = CASES[case]
    print(f"[case] noalloc {name} {first} then {second}", flush=True)
    rng = np.random.default_rng(case)
    for (m, k, n, variant), act in ((first, RELU), (second, LINEAR)):
        _both(rng, m, k, n, act, variant)


def test_noalloc_refuses_more_than_its_scratch(gpu):
    # bf16 planes of 8192 x 8192 activations: 128 MiB > 64 MiB
    rng = np.random.default_rng(9)
    m = k = n = 8192
    codes, scale = _weights(rng, n, k)
    x = DeviceArray.from_numpy(np.zeros((m, k), np.float32))
    y = DeviceArray.from_numpy(np.full((m, n), 7.0, np.float32))
    with pytest.raises(ValueError, match="scratch"):
        _call("enq_dense_w8_noalloc", x, m, k, codes, scale, n, None, LINEAR, _lib.W8_BF16, y,
              None)
    assert np.all(y.numpy() == 7.0)
    # the library still works afterwards
    _both(rng, 8, 256, 64, LINEAR, _lib.W8_FP32)
