"""GPU parity of the QAT forward (``Enilnets/graph/quantization.py:94-141``).

* The per-step fake-quantized weight is bit-identical to the oracle's
  (per channel and per tensor, several bit widths).
* ``forward`` is within the Dense bound of the float64 product with that
  weight; with activation quantization, the observer's moving range follows
  the oracle's observer fed the same outputs, and outputs sit within one
  grid step of the oracle's.
"""

import numpy as np
import pytest

from enilnets_amd.device import DeviceArray
from enilnets_amd.nn.qat import QATLinear
import oracle

pytestmark = pytest.mark.gpu


def row_rel_err(got, ref):
    denom = np.maximum(np.max(np.abs(ref), axis=-1), 1e-30)
    return np.max(np.abs(np.asarray(got, np.float64) - ref), axis=-1) / denom


@pytest.mark.parametrize("bits,per_channel", [(8, True), (8, False), (4, True), (6, False)])
def test_quantized_weight_bit_exact(gpu, bits, per_channel):
    rng = np.random.default_rng(bits)
    w = (rng.standard_normal((96, 200)) * 0.1).astype(np.float32)
    layer = QATLinear.from_weights(w, bits=bits, per_channel=per_channel)
    fake, _ = layer.quantized_weight()
    want = oracle.qat_quantized_weight(w, bits, per_channel)
    assert np.array_equal(fake.numpy().view(np.uint32), want.view(np.uint32))


def test_forward_and_training_steps(gpu):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 128)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(64) * 0.01).astype(np.float32)
    layer = QATLinear.from_weights(w, b)
    x = rng.standard_normal((300, 128)).astype(np.float32)
    y = layer.forward(DeviceArray.from_numpy(x)).numpy()
    want = x.astype(np.float64) @ oracle.qat_quantized_weight(w).T.astype(np.float64) + b
    assert np.all(row_rel_err(y, want) <= 1e-4)
    # a training update changes the grid the next forward uses
    w2 = w - 0.05 * np.sign(w)
    layer.load_weight(w2)
    y2 = layer.forward(DeviceArray.from_numpy(x)).numpy()
    want2 = x.astype(np.float64) @ oracle.qat_quantized_weight(w2).T.astype(np.float64) + b
    assert np.all(row_rel_err(y2, want2) <= 1e-4)


def test_activation_quantization_observer(gpu):
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((32, 64)) * 0.2).astype(np.float32)
    b = np.zeros(32, np.float32)
    layer = QATLinear.from_weights(w, b, quantize_activations=True)
    obs = oracle.MovingRange()
    for step in range(3):
        x = rng.standard_normal((128, 64)).astype(np.float32)
        raw = layer.forward(DeviceArray.from_numpy(x), training=False) if step else None
        y = layer.forward(DeviceArray.from_numpy(x), training=True).numpy()
        plain = x.astype(np.float64) @ oracle.qat_quantized_weight(w).T.astype(np.float64)
        obs.observe(plain.astype(np.float32))
        assert abs(layer.observer.low - obs.low) <= 1e-4 * abs(obs.low)
        assert abs(layer.observer.high - obs.high) <= 1e-4 * abs(obs.high)
        s, z = obs.scale_and_zero_point(8, "asymmetric")
        want = oracle.fake_quantize(plain.astype(np.float32), s, z, 8, "asymmetric")
        assert np.all(np.abs(y - want) <= 1.01 * float(s))
        del raw


def test_reference_constructor(gpu):
    # QATLinear(n_in, n_out, ...) as graph/quantization.py:106-117 builds it:
    # init_weights(n_in, n_out) weights (n_out, n_in), zero bias
    from enilnets_amd.nn.weight_init import init_weights
    np.random.seed(21)
    layer = QATLinear(128, 48, bits=8, quantize_activations=False)
    np.random.seed(21)
    w, b = init_weights(128, 48, "xavier_uniform")
    assert layer.weight.shape == (48, 128)
    assert np.array_equal(layer.weight.numpy(), w) and not layer.bias.numpy().any()
    x = np.random.default_rng(2).standard_normal((32, 128)).astype(np.float32)
    y = layer.forward(DeviceArray.from_numpy(x), training=False).numpy()
    fq = oracle.qat_quantized_weight(w, 8, True)
    want = x.astype(np.float64) @ fq.astype(np.float64).T
    assert np.all(row_rel_err(y, want) <= 1e-4)
    with pytest.raises(ValueError):
        QATLinear(8, 8, init_method="nope")
