"""GPU round trip of the int8 on-disk format (``enilnets_amd.nn.io``).

The reference's ``Save`` keeps fake-quantized floats (``nn/io.py:61-112``);
this format keeps int8 codes and the ``quant`` specs.  Loading must give back
every layer value bit for bit (the fake-quantized weights are rebuilt as
``code * scale`` in float32, which is how ``dequantize`` forms them), the
same device codes, and therefore the same ``Forward`` output bit for bit;
the int8 weights take a quarter of their float32 bytes.
"""

import os

import numpy as np
import pytest

import enilnets_amd as ea
from enilnets_amd.nn import LoadInt8, Model, SaveInt8, int8_weights

pytestmark = pytest.mark.gpu


def model_with_everything(rng):
    m = Model()
    E, H = 64, 4
    ws = [(rng.standard_normal((E, E)) * 0.05).astype(np.float32) for _ in range(4)]
    m.add_residual_start()
    m.add_layernorm(E)
    m.add_multihead_attention(*ws, num_heads=H, causal=True)
    m.add_residual_end()
    m.add_dense((rng.standard_normal((128, E)) * 0.05).astype(np.float32),
                (rng.standard_normal(128) * 0.01).astype(np.float32), "gelu")
    m.add_moe((rng.standard_normal((4, 96, 128)) * 0.05).astype(np.float32),
              (rng.standard_normal((4, 128, 96)) * 0.05).astype(np.float32),
              (rng.standard_normal((4, 128)) * 0.1).astype(np.float32), top_k=2)
    m.add_dense((rng.standard_normal((10, 128)) * 0.05).astype(np.float32),
                np.zeros(10, np.float32), "linear")
    return m


@pytest.mark.parametrize("per_channel", [True, False])
def test_int8_round_trip(gpu, tmp_path, per_channel):
    rng = np.random.default_rng(int(per_channel))
    m = model_with_everything(rng)
    ea.quantize_weights(m, per_channel=per_channel)
    x = rng.standard_normal((2, 16, 64)).astype(np.float32)
    cal = ea.ActivationCalibrator(m)
    cal.observe(x)
    cal.apply()
    y = m.Forward(x)
    f = str(tmp_path / "model.int8")
    info = SaveInt8(m, f)
    assert info["int8_bytes"] * 4 == info["float_bytes"]
    assert os.path.getsize(f) < 0.35 * info["float_bytes"] + 200_000
    m2 = LoadInt8(f)
    for a, b in zip(m.layers, m2.layers):
        assert [k for k in a if not k.startswith("_state_")] == list(b)
        for k, v in b.items():
            if isinstance(v, np.ndarray):
                assert v.dtype == a[k].dtype and v.shape == a[k].shape, k
                assert np.array_equal(v.view(np.uint8), a[k].view(np.uint8)), k
        for name, spec in b.get("quant", {}).items():
            for field, val in spec.items():
                ref = a["quant"][name][field]
                assert type(val) is type(ref) and np.array_equal(val, ref), (name, field)
        for key in b.get("quant", {}):
            if key in b.get("_state_enq_int8", {}):
                c1 = int8_weights(a, key).codes.numpy()
                c2 = int8_weights(b, key).codes.numpy()
                assert np.array_equal(c1, c2), key
    y2 = m2.Forward(x)
    assert y2.dtype == y.dtype and np.array_equal(y2, y)
