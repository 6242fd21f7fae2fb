"""NumPy restatement of the quantization-aware-training forward.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Follows
``Enilnets/graph/quantization.py``: ``QATLinear.quantized_weight``
(``:119-130``), ``QATLinear.forward`` (``:132-141``), the moving-average
observer (``:61-91``) and the straight-through mask (``:31-40``).
"""

from typing import Any, Optional, Tuple

import numpy as np

from .quantization import compute_scale, fake_quantize, quant_range


def qat_quantized_weight(w: Any, bits: int = 8, per_channel: bool = True) -> Any:
    """Symmetric fake quantization of ``w`` per output channel (min / max
    over every axis but 0, keepdims) or per tensor."""
    w = np.asarray(w)
    if per_channel and w.ndim > 1:
        axes = tuple(range(1, w.ndim))
        low = np.min(w, axis=axes, keepdims=True)
        high = np.max(w, axis=axes, keepdims=True)
    else:
        low, high = np.min(w), np.max(w)
    scale, zero_point = compute_scale(low, high, bits, "symmetric")
    return fake_quantize(w, scale, zero_point, bits, "symmetric")


class MovingRange:
    """``MovingRangeObserver``: EMA of min / max with Python floats."""

    def __init__(self, momentum: float = 0.9) -> None:
        self.momentum = momentum
        self.low: Optional[float] = None
        self.high: Optional[float] = None

    def observe(self, x: Any) -> None:
        low, high = float(np.min(x)), float(np.max(x))
        if self.low is None:
            self.low, self.high = low, high
        else:
            m = self.momentum
            self.low = m * self.low + (1 - m) * low
            self.high = m * self.high + (1 - m) * high

    def scale_and_zero_point(self, bits: int, scheme: str) -> Tuple[Any, Any]:
        return compute_scale(np.asarray(self.low), np.asarray(self.high), bits, scheme)


def qat_linear_forward(w: Any, b: Any, x: Any, bits: int = 8, per_channel: bool = True,
                       observer: Optional[MovingRange] = None, act_bits: int = 8,
                       training: bool = True) -> Any:
    """``x @ fq(W).T + b``; with an observer, its activation fake-quant."""
    out = np.matmul(x, qat_quantized_weight(w, bits, per_channel).T) + b
    if observer is None:
        return out
    if training:
        observer.observe(out)
    scale, zero_point = observer.scale_and_zero_point(act_bits, "asymmetric")
    return fake_quantize(out, scale, zero_point, act_bits, "asymmetric")


def ste_mask(x: Any, scale: Any, zero_point: Any, bits: int, scheme: str) -> Any:
    """Pass-through region of the straight-through backward."""
    qmin, qmax = quant_range(bits, scheme)
    return (x >= (qmin - zero_point) * scale) & (x <= (qmax - zero_point) * scale)
