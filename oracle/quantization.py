"""NumPy restatement of Enilnets' post-training quantization primitives.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): never imported by the
product package.

Every function follows one function of the reference module
``Enilnets/compression/quantization.py`` (cited per function).  The
arithmetic is kept in the reference's order because the HIP kernels are
checked against it bit for bit:

* the symmetric scale is ``amax / qmax`` with a true (correctly rounded)
  division, replaced by 1.0 where ``amax`` is not positive (NaN included);
* codes are ``clip(round_half_even(x / scale + zero_point), qmin, qmax)``,
  with the ``+ zero_point`` done before rounding (it turns ``-0.0`` into
  ``+0.0`` before the round, while small negatives still round to ``-0.0``);
* dequantization is ``(q - zero_point) * scale``;
* the input dtype is preserved (float64 stays float64).
"""

from typing import Any, Dict, Optional, Sequence, Tuple

import numpy as np


def quant_range(bits: int, scheme: str) -> Tuple[int, int]:
    """Integer grid for ``bits`` under ``scheme``.

    Follows ``compression/quantization.py:21-30``: bits outside [2, 16] and
    unknown schemes raise ValueError; symmetric is ``[-(2^(b-1)-1),
    2^(b-1)-1]``, asymmetric ``[0, 2^b - 1]``."""
    if bits < 2 or bits > 16:
        raise ValueError(f"bits must be between 2 and 16, got {bits}")
    if scheme == "symmetric":
        top = (1 << (bits - 1)) - 1
        return -top, top
    if scheme == "asymmetric":
        return 0, (1 << bits) - 1
    raise ValueError(f"scheme must be 'symmetric' or 'asymmetric', got {scheme!r}")


def compute_scale(low: Any, high: Any, bits: int, scheme: str) -> Tuple[Any, Any]:
    """Scale and zero point for the range [low, high].

    Follows ``compression/quantization.py:33-50``."""
    qmin, qmax = quant_range(bits, scheme)
    if scheme == "symmetric":
        magnitude = np.maximum(np.abs(low), np.abs(high))
        scale = np.where(magnitude > 0, magnitude / qmax, 1.0)
        return scale, np.zeros_like(scale)
    width = high - low
    scale = np.where(width > 0, width / (qmax - qmin), 1.0)
    return scale, np.round(qmin - low / scale)


def quantize(x: Any, scale: Any, zero_point: Any, bits: int, scheme: str) -> Any:
    """Float codes on the integer grid.  Follows
    ``compression/quantization.py:53-56``."""
    qmin, qmax = quant_range(bits, scheme)
    shifted = x / scale + zero_point
    return np.clip(np.round(shifted), qmin, qmax)


def dequantize(q: Any, scale: Any, zero_point: Any) -> Any:
    """Codes back to floats.  Follows ``compression/quantization.py:59-61``."""
    return (q - zero_point) * scale


def fake_quantize(x: Any, scale: Any, zero_point: Any, bits: int, scheme: str) -> Any:
    """Round-trip through the grid.  Follows
    ``compression/quantization.py:64-69``."""
    codes = quantize(x, scale, zero_point, bits, scheme)
    return dequantize(codes, scale, zero_point)


def _reduce_axes(ndim: int, keep: int) -> Tuple[int, ...]:
    # compression/quantization.py:72-73: every axis except the kept one.
    return tuple(a for a in range(ndim) if a != keep)


def quantize_tensor(w: Any, bits: int = 8, scheme: str = "symmetric",
                    per_channel: bool = False, axis: int = 0) -> Tuple[Any, Any, Any]:
    """``(fake_quantized, scale, zero_point)`` of one tensor.

    Follows ``compression/quantization.py:76-93``: per-channel statistics
    only when the tensor has more than one dimension, reduced over every
    axis except ``axis`` with keepdims; otherwise one global min/max."""
    w = np.asarray(w)
    if per_channel and w.ndim > 1:
        axes = _reduce_axes(w.ndim, axis)
        low = w.min(axis=axes, keepdims=True)
        high = w.max(axis=axes, keepdims=True)
    else:
        low = np.min(w)
        high = np.max(w)
    scale, zero_point = compute_scale(low, high, bits, scheme)
    return fake_quantize(w, scale, zero_point, bits, scheme), scale, zero_point


def int8_codes(w: Any, per_channel: bool = True) -> Tuple[np.ndarray, Any]:
    """Symmetric 8-bit codes as int8 plus the float scale.

    Not a reference function: the reference never materialises int8
    (``compression/quantization.py:1-14``).  It is the reference's own
    ``quantize`` (``:53-56``) with the scale of ``quantize_tensor``
    (``:76-93``), cast to int8.  The cast is exact because the codes are
    integers in [-127, 127]."""
    w = np.asarray(w)
    _, scale, zero_point = quantize_tensor(w, 8, "symmetric", per_channel)
    codes = quantize(w, scale, zero_point, 8, "symmetric")
    return codes.astype(np.int8), scale


#: Follows ``compression/quantization.py:99-112``: which parameters of each
#: layer type are quantized.
QUANTIZABLE = {
    "dense": ("weights",),
    "sparse": ("weights",),
    "conv2d": ("weights",),
    "conv1d": ("weights",),
    "embedding": ("weights",),
    "multihead_attention": ("Wq", "Wk", "Wv", "Wo"),
    "cross_attention": ("Wq", "Wk", "Wv", "Wo"),
    "rnn": ("Wx", "Wh"),
    "lstm": ("Wx", "Wh"),
    "gru": ("Wx", "Wh"),
    "moe": ("W1", "W2", "Wr"),
    "cbam_channel": ("W1", "W2"),
}


def quantize_weights(model: Any, bits: int = 8, scheme: str = "symmetric",
                     per_channel: bool = False,
                     layer_types: Optional[Sequence[str]] = None) -> Dict[str, Any]:
    """In-place post-training quantization of ``model.layers``.

    Follows ``compression/quantization.py:115-153``: layer order, the
    ``layer_types`` filter, the ``QUANTIZABLE`` table, the in-place write of
    the fake-quantized array, the ``quant`` spec and the report fields."""
    report: Dict[str, Any] = {"bits": bits, "scheme": scheme,
                              "per_channel": per_channel, "layers": {}}
    weighted_err = 0.0
    count = 0
    float_bytes = 0
    packed_bits = 0
    for index, layer in enumerate(model.layers):
        if layer_types is not None and layer["type"] not in layer_types:
            continue
        for name in QUANTIZABLE.get(layer["type"], ()):
            if name not in layer:
                continue
            source = layer[name]
            fq, scale, zero_point = quantize_tensor(source, bits, scheme, per_channel)
            err = float(np.mean(np.abs(fq - source)))
            layer[name] = fq
            layer.setdefault("quant", {})[name] = {
                "bits": bits, "scheme": scheme,
                "scale": scale, "zero_point": zero_point}
            size = int(source.size)
            report["layers"][f"{index}.{name}"] = {"mean_abs_error": err, "size": size}
            weighted_err += err * source.size
            count += size
            float_bytes += size * source.dtype.itemsize
            packed_bits += size * bits
    report["mean_abs_error"] = weighted_err / count if count else 0.0
    report["parameters"] = count
    report["float_bytes"] = float_bytes
    report["quantized_bytes"] = packed_bits // 8
    report["compression"] = (float_bytes / (packed_bits / 8)) if packed_bits else 1.0
    return report


def quantization_error(reference: Sequence[Any], candidate: Sequence[Any]) -> Dict[str, float]:
    """Mean / max absolute error and relative L2 of two output sets.

    Follows ``compression/quantization.py:218-229``."""
    a = np.concatenate([np.asarray(v).reshape(-1) for v in reference])
    b = np.concatenate([np.asarray(v).reshape(-1) for v in candidate])
    diff = b - a
    norm = float(np.sqrt(np.sum(a * a)))
    rel = float(np.sqrt(np.sum(diff * diff)) / norm) if norm > 0 else 0.0
    return {"mean_abs_error": float(np.mean(np.abs(diff))),
            "max_abs_error": float(np.max(np.abs(diff))),
            "relative_error": rel}
