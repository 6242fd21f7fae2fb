"""Quantization-aware-training forward on the device
(``Enilnets/graph/quantization.py:55-141``).

``QATLinear.forward`` re-quantizes its weight per output channel on every
call (one ``enq_quantize_tensor`` pass gives the fake-quantized weight, its
int8 codes and scales), then runs ``x . fq(W)^T + b`` as a W8 Dense on those
codes -- the product with the fake-quantized weight, since ``fq(W) = code *
scale``.  With ``quantize_activations`` the output is fake-quantized with the
moving-average range of ``MovingRangeObserver`` (updated in training mode,
read in eval mode).  The straight-through backward (``:31-40``) belongs to
the reference's autograd and stays there; ``ste_mask`` gives its mask.
"""

from typing import Any, Optional, Tuple

import numpy as np

from .. import _lib
from ..device import DeviceArray, null
from .dense import act_quant, dense_w8
from .weights import Int8Weights


class MovingRangeObserver:
    """Exponential moving average of a tensor's min / max
    (``graph/quantization.py:61-91``)."""

    def __init__(self, momentum: float = 0.9) -> None:
        if not 0.0 <= momentum < 1.0:
            raise ValueError(f"momentum must be in [0, 1), got {momentum}")
        self.momentum = momentum
        self.low: Optional[float] = None
        self.high: Optional[float] = None

    def observe(self, x: DeviceArray) -> None:
        d_lo, d_hi = DeviceArray((1,), np.float32), DeviceArray((1,), np.float32)
        _lib.call("enq_minmax", _lib.F32, x.ptr, 1, 1, x.size, d_lo.ptr, d_hi.ptr)
        low, high = float(d_lo.numpy()[0]), float(d_hi.numpy()[0])
        if self.low is None:
            self.low, self.high = low, high
        else:
            m = self.momentum
            self.low = m * self.low + (1 - m) * low
            self.high = m * self.high + (1 - m) * high

    def scale_and_zero_point(self, bits: int, scheme: str) -> Tuple[Any, Any]:
        from ..compression.quantization import compute_scale
        if self.low is None:
            raise RuntimeError("observer has seen no data yet")
        return compute_scale(np.asarray(self.low), np.asarray(self.high), bits, scheme)


class QATLinear:
    """Device twin of ``graph.quantization.QATLinear`` (``:94-141``) for the
    forward pass.  ``QATLinear(n_in, n_out, ...)`` takes the reference's
    arguments (``:106-117``: ``init_weights(n_in, n_out, init_method)``, a
    ``(n_out, n_in)`` weight and zero bias); ``QATLinear.from_weights``
    starts from given float32 arrays."""

    def __init__(self, n_in: int, n_out: int, bits: int = 8, per_channel: bool = True,
                 quantize_activations: bool = False, act_bits: int = 8,
                 init_method: str = "xavier_uniform") -> None:
        from .weight_init import init_weights
        w, b = init_weights(int(n_in), int(n_out), method=init_method)
        self._setup(w, b, bits, per_channel, quantize_activations, act_bits)

    @classmethod
    def from_weights(cls, weight: Any, bias: Any = None, bits: int = 8, per_channel: bool = True,
                     quantize_activations: bool = False, act_bits: int = 8) -> "QATLinear":
        """A layer with weight ``(n_out, n_in)`` and bias ``(n_out,)`` (zero when None)."""
        self = cls.__new__(cls)
        w = np.asarray(weight, dtype=np.float32)
        if w.ndim != 2:
            raise ValueError(f"QATLinear weight must be 2-D, got {w.shape}")
        b = np.zeros(w.shape[0], np.float32) if bias is None else bias
        self._setup(w, b, bits, per_channel, quantize_activations, act_bits)
        return self

    def _setup(self, w: np.ndarray, b: Any, bits: int, per_channel: bool,
               quantize_activations: bool, act_bits: int) -> None:
        w = np.ascontiguousarray(w, dtype=np.float32)
        if not 2 <= int(bits) <= 8:
            raise NotImplementedError("the device QAT forward takes 2- to 8-bit weights")
        self.weight = DeviceArray.from_numpy(w)
        self.bias = DeviceArray.from_numpy(np.ascontiguousarray(b, dtype=np.float32))
        self.bits, self.act_bits = int(bits), int(act_bits)
        self.per_channel = per_channel
        self.quantize_activations = quantize_activations
        self.observer = MovingRangeObserver()

    def load_weight(self, weight: Any) -> None:
        """Copy updated (e.g. trained) weights in."""
        self.weight.copy_from(np.asarray(weight, dtype=np.float32))

    def quantized_weight(self) -> Tuple[DeviceArray, Int8Weights]:
        """``(fq(W), int8 weights)``: symmetric fake quantization per output
        channel (``:119-130``), or per tensor."""
        n_out, n_in = self.weight.shape
        channels, inner = (n_out, n_in) if self.per_channel else (1, n_out * n_in)
        fake = DeviceArray(self.weight.shape, np.float32)
        codes = DeviceArray(self.weight.shape, np.int8)
        scale = DeviceArray((channels,), np.float32)
        zp = DeviceArray((channels,), np.float32)
        _lib.call("enq_quantize_tensor", _lib.F32, self.weight.ptr, 1, channels, inner,
                  self.bits, _lib.SYMMETRIC, fake.ptr, codes.ptr, scale.ptr, zp.ptr, null())
        if not self.per_channel:
            one = float(scale.numpy()[0])
            scale = DeviceArray.from_numpy(np.full(n_out, one, np.float32))
        return fake, Int8Weights(codes, scale, self.weight.shape, self.bits, self.per_channel,
                                 None, None)

    def forward(self, x: DeviceArray, training: bool = True,
                variant: str = "fp32") -> DeviceArray:
        """``:132-141``: ``x . fq(W)^T + b``, then the activation
        fake-quantization when enabled."""
        _, wq = self.quantized_weight()
        out = dense_w8(x, wq, self.bias, "linear", variant=variant)
        if not self.quantize_activations:
            return out
        if training:
            self.observer.observe(out)
        scale, zero_point = self.observer.scale_and_zero_point(self.act_bits, "asymmetric")
        spec = {"bits": self.act_bits, "scheme": "asymmetric", "scale": scale,
                "zero_point": zero_point}
        return act_quant(out, spec, np.float32)

    __call__ = forward


def ste_mask(x: np.ndarray, scale: Any, zero_point: Any, bits: int, scheme: str) -> np.ndarray:
    """The straight-through estimator's pass-through mask (``:31-40``):
    True inside the representable range ``[(qmin - zp) s, (qmax - zp) s]``."""
    from ..compression.quantization import quant_range
    qmin, qmax = quant_range(bits, scheme)
    low = (qmin - zero_point) * scale
    high = (qmax - zero_point) * scale
    return (x >= low) & (x <= high)
