"""Captured graphs of library calls replay the eager results exactly."""

import ctypes

import numpy as np
import pytest

from enilnets_amd import _lib
from enilnets_amd.device import DeviceArray
from enilnets_amd.graph import capture
from enilnets_amd.nn import transformer as T
from enilnets_amd.nn.dense import dense_w8, quantize_weight_rows

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(gpu):
    # LayerNorm, a W8 Dense and a residual add, captured once and replayed
    # three times with other eager work and synchronisations between the
    # replays; the output is cleared before each replay
    print("[case] graph of layernorm + dense_w8 + add", flush=True)
    rng = np.random.default_rng(3)
    m, e = 512, 256
    layer = {"gamma": np.ones(e, np.float32), "beta": np.zeros(e, np.float32), "epsilon": 1e-5}
    w = quantize_weight_rows(rng.normal(0.0, 0.05, (e, e)).astype(np.float32))
    x = DeviceArray.from_numpy(rng.standard_normal((m, e)).astype(np.float32))
    params = T.layernorm_params(layer)
    t, h, y = (DeviceArray((m, e), np.float32) for _ in range(3))

    def seq():
        T.layernorm(x, layer, out=t, params=params)
        dense_w8(t, w, None, "gelu", out=h)
        T.residual_add(h, x, out=y)

    seq()
    want = y.numpy()
    other = DeviceArray.from_numpy(rng.standard_normal((m, e)).astype(np.float32))
    g = capture(seq)
    try:
        for _ in range(3):
            zeros = np.zeros((m, e), np.float32)
            _lib.call("enq_copy_to_device", y.ptr, zeros.ctypes.data_as(ctypes.c_void_p),
                      ctypes.c_size_t(zeros.nbytes))
            g.replay()
            assert np.array_equal(y.numpy(), want)
            dense_w8(other, w, None, "relu")   # eager work between replays
            _lib.synchronize()
    finally:
        g.close()


def test_graph_keeps_workspace(gpu):
    # while a graph is alive a call needing a larger workspace fails cleanly
    print("[case] graph workspace growth refused", flush=True)
    w = quantize_weight_rows(np.full((64, 64), 0.01, np.float32))
    x = DeviceArray.from_numpy(np.ones((128, 64), np.float32))
    y = DeviceArray((128, 64), np.float32)
    seq = lambda: dense_w8(x, w, None, "linear", out=y)
    seq()
    big_w = quantize_weight_rows(np.full((8192, 8192), 0.01, np.float32))
    big_x = DeviceArray((65536, 8192), np.float32)   # never read: the call fails first
    g = capture(seq)
    try:
        with pytest.raises(ValueError, match="captured graph"):
            dense_w8(big_x, big_w, None, "linear")
    finally:
        g.close()
