"""Drop-in replacement for ``Enilnets.compression.quantization`` on MI355X.

Same functions, same arguments, same NumPy arrays in and out as the
reference module (``Enilnets/compression/quantization.py``); the arithmetic
runs in HIP kernels of libenilnets_amd and is bit-identical to the reference
for float32 and float64 tensors (round half to even, true division, NaN and
-0.0 behaviour included).

Output dtypes and container types (0-d array vs. NumPy scalar) follow NumPy
2's promotion rules, which the reference inherits; they are resolved by
evaluating the reference's expression on size-1 probe values, which fixes
only metadata and never the numbers returned.

There is no CPU fallback.  Tensors of a dtype the kernels do not cover
(float16, complex) raise NotImplementedError.
"""

import ctypes
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from .. import _lib
from ..device import DeviceArray, null

__all__ = [
    "quant_range", "compute_scale", "quantize", "dequantize", "fake_quantize",
    "quantize_tensor", "QUANTIZABLE", "quantize_weights", "quantization_error",
    "ActivationCalibrator", "remove_activation_quantization",
]

_CODES = {np.dtype(np.float32): _lib.F32, np.dtype(np.float64): _lib.F64}


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _probe(v: Any) -> Any:
    """A stand-in for ``v`` with its promotion behaviour (Python scalars stay
    weak, arrays and NumPy scalars keep their dtype) and value 1."""
    if isinstance(v, (bool, int, float)) and not isinstance(v, np.generic):
        return type(v)(1)
    a = np.asarray(v)
    return np.ones((), dtype=a.dtype)


def _compute_code(dtype: np.dtype) -> int:
    dtype = np.dtype(dtype)
    if dtype not in _CODES:
        raise NotImplementedError(
            f"enilnets_amd computes in float32 or float64; dtype {dtype} is not supported")
    return _CODES[dtype]


def _shape_of(v: Any) -> Tuple[int, ...]:
    return tuple(np.shape(v))


def _channel_layout(out_shape: Tuple[int, ...], params: Sequence[Any], dtype: np.dtype):
    """Map per-channel parameters broadcast against ``out_shape`` to the
    kernels' (outer, channels, inner) layout.

    Returns ``(outer, channels, inner, [flat parameter arrays])``.  The axes
    along which any parameter varies are merged into one channel block when
    they are contiguous; otherwise every element is its own channel."""
    nd = len(out_shape)
    padded = []
    varying = set()
    for p in params:
        a = np.asarray(p)
        shape = (1,) * (nd - a.ndim) + a.shape
        padded.append(a.reshape(shape))
        for ax, (d, o) in enumerate(zip(shape, out_shape)):
            if d != 1 and o != 1:
                varying.add(ax)
    total = int(np.prod(out_shape, dtype=np.int64))
    if not varying:
        flats = [np.ascontiguousarray(p.reshape(-1)[:1], dtype=dtype) for p in padded]
        return 1, 1, total, flats
    lo, hi = min(varying), max(varying) + 1
    block = out_shape[lo:hi]
    sel = tuple(slice(None) if lo <= ax < hi else 0 for ax in range(nd))
    flats = [np.ascontiguousarray(np.broadcast_to(p[sel], block).reshape(-1), dtype=dtype)
             for p in padded]
    outer = int(np.prod(out_shape[:lo], dtype=np.int64))
    channels = int(np.prod(block, dtype=np.int64))
    inner = int(np.prod(out_shape[hi:], dtype=np.int64))
    return outer, channels, inner, flats


def _as_container(values: np.ndarray, like: Any) -> Any:
    """A 0-d result takes the container of ``like`` (NumPy scalar or 0-d
    ndarray, which NumPy's functions choose differently); anything larger is
    an ndarray."""
    if values.ndim > 0 or isinstance(like, np.ndarray):
        return values
    return values.reshape(())[()]


def _scale_like(pl: Any, ph: Any, bits: int, scheme: str) -> Tuple[Any, Any]:
    """compute_scale's expression (``quantization.py:41-50``) on probe values:
    fixes the dtype and container of the scale and zero point."""
    qmin, qmax = quant_range(bits, scheme)
    if scheme == "symmetric":
        m = np.maximum(np.abs(pl), np.abs(ph))
        s_like = np.where(m > 0, m / qmax, 1.0)
        return s_like, np.zeros_like(s_like)
    s_like = np.where((ph - pl) > 0, (ph - pl) / (qmax - qmin), 1.0)
    return s_like, np.round(qmin - pl / s_like)


# ---------------------------------------------------------------------------
# the reference's module functions
# ---------------------------------------------------------------------------
def quant_range(bits: int, scheme: str) -> Tuple[int, int]:
    """Integer interval ``bits`` at ``scheme`` maps onto.

    Same contract as ``compression/quantization.py:21-30`` (ValueError for
    bits outside [2, 16] or an unknown scheme).  Pure host logic."""
    if not 2 <= bits <= 16:
        raise ValueError(f"bits must be between 2 and 16, got {bits}")
    if scheme == "symmetric":
        return -(2 ** (bits - 1) - 1), 2 ** (bits - 1) - 1
    if scheme == "asymmetric":
        return 0, 2 ** bits - 1
    raise ValueError(f"scheme must be 'symmetric' or 'asymmetric', got {scheme!r}")


def _scheme_code(scheme: str) -> int:
    return _lib.SYMMETRIC if scheme == "symmetric" else _lib.ASYMMETRIC


def compute_scale(low: Any, high: Any, bits: int, scheme: str) -> Tuple[Any, Any]:
    """Scale and zero point mapping ``[low, high]`` onto the integer grid.

    Replaces ``compression/quantization.py:33-50``; computed by
    ``enq_compute_scale``."""
    quant_range(bits, scheme)
    s_like, z_like = _scale_like(_probe(low), _probe(high), bits, scheme)
    dtype = np.result_type(s_like)
    code = _compute_code(dtype)
    shape = np.broadcast_shapes(_shape_of(low), _shape_of(high))
    lo = np.ascontiguousarray(np.broadcast_to(np.asarray(low), shape), dtype=dtype)
    hi = np.ascontiguousarray(np.broadcast_to(np.asarray(high), shape), dtype=dtype)
    n = lo.size
    scale = np.empty(shape, dtype)
    zp = np.empty(shape, np.result_type(z_like))
    if n:
        d_lo, d_hi = DeviceArray.from_numpy(lo), DeviceArray.from_numpy(hi)
        d_s, d_z = DeviceArray(shape, dtype), DeviceArray(shape, dtype)
        _lib.call("enq_compute_scale", code, d_lo.ptr, d_hi.ptr, n, bits, _scheme_code(scheme),
                  d_s.ptr, d_z.ptr)
        scale = d_s.numpy()
        zp = d_z.numpy().astype(zp.dtype, copy=False)
    return _as_container(scale, s_like), _as_container(zp, z_like)


def _elementwise(entry: str, x: Any, scale: Any, zero_point: Any, like: Any,
                 qmin: int = 0, qmax: int = 0) -> Any:
    """Run one of the broadcasting elementwise kernels."""
    dtype = np.result_type(like)
    code = _compute_code(dtype)
    out_shape = np.broadcast_shapes(_shape_of(x), _shape_of(scale), _shape_of(zero_point))
    out = np.empty(out_shape, dtype)
    if out.size == 0:
        return _as_container(out, like)
    xb = np.ascontiguousarray(np.broadcast_to(np.asarray(x), out_shape), dtype=dtype)
    outer, channels, inner, (s, z) = _channel_layout(out_shape, (scale, zero_point), dtype)
    d_x = DeviceArray.from_numpy(xb)
    d_s, d_z = DeviceArray.from_numpy(s), DeviceArray.from_numpy(z)
    d_out = DeviceArray(out_shape, dtype)
    if entry == "enq_dequantize":
        _lib.call(entry, code, d_x.ptr, outer, channels, inner, d_s.ptr, d_z.ptr, d_out.ptr)
    else:
        _lib.call(entry, code, d_x.ptr, outer, channels, inner, d_s.ptr, d_z.ptr, qmin, qmax,
                  d_out.ptr)
    return _as_container(d_out.numpy(), like)


def quantize(x: Any, scale: Any, zero_point: Any, bits: int, scheme: str) -> Any:
    """Float -> integer codes, clipped to the representable range.

    Replaces ``compression/quantization.py:53-56`` (``enq_quantize``)."""
    qmin, qmax = quant_range(bits, scheme)
    like = np.clip(np.round(_probe(x) / _probe(scale) + _probe(zero_point)), qmin, qmax)
    return _elementwise("enq_quantize", x, scale, zero_point, like, qmin, qmax)


def dequantize(q: Any, scale: Any, zero_point: Any) -> Any:
    """Integer codes -> the float values they stand for.

    Replaces ``compression/quantization.py:59-61`` (``enq_dequantize``)."""
    like = (_probe(q) - _probe(zero_point)) * _probe(scale)
    return _elementwise("enq_dequantize", q, scale, zero_point, like)


def fake_quantize(x: Any, scale: Any, zero_point: Any, bits: int, scheme: str) -> Any:
    """Round ``x`` onto the integer grid and back in one kernel.

    Replaces ``compression/quantization.py:64-69`` (``enq_fake_quantize``)."""
    qmin, qmax = quant_range(bits, scheme)
    ps, pz = _probe(scale), _probe(zero_point)
    codes = np.clip(np.round(_probe(x) / ps + pz), qmin, qmax)
    like = (codes - pz) * ps
    return _elementwise("enq_fake_quantize", x, scale, zero_point, like, qmin, qmax)


def _tensor_layout(w: np.ndarray, per_channel: bool, axis: int):
    """(outer, channels, inner, scale shape) of quantize_tensor's reduction
    (``compression/quantization.py:86-91``).  An ``axis`` outside
    [0, ndim) matches no axis there, so every axis is reduced (keepdims)."""
    if per_channel and w.ndim > 1:
        if 0 <= axis < w.ndim:
            outer = int(np.prod(w.shape[:axis], dtype=np.int64))
            channels = int(w.shape[axis])
            inner = int(np.prod(w.shape[axis + 1:], dtype=np.int64))
            sshape = tuple(w.shape[a] if a == axis else 1 for a in range(w.ndim))
            return outer, channels, inner, sshape
        return 1, 1, int(w.size), (1,) * w.ndim
    return 1, 1, int(w.size), ()


def _compute_dtype_for_tensor(w: np.ndarray) -> np.dtype:
    if w.dtype.kind in "biu":
        return np.dtype(np.float64)     # the reference's integer path promotes to float64
    _compute_code(w.dtype)
    return w.dtype


def _quantize_tensor_device(w: np.ndarray, bits: int, scheme: str, per_channel: bool,
                            axis: int, want_codes: bool, want_err: bool):
    """Run ``enq_quantize_tensor``; returns host (fake, scale, zp), the device
    codes (or None), the device scale and the |error| sum (or None)."""
    dtype = _compute_dtype_for_tensor(w)
    code = _compute_code(dtype)
    outer, channels, inner, sshape = _tensor_layout(w, per_channel, axis)
    src = np.ascontiguousarray(w, dtype=dtype)
    d_w = DeviceArray.from_numpy(src)
    d_fake = DeviceArray(w.shape, dtype)
    d_codes = DeviceArray(w.shape, np.int8) if want_codes else None
    d_s = DeviceArray((channels,), dtype)
    d_z = DeviceArray((channels,), dtype)
    err = ctypes.c_double(0.0)
    d_err = DeviceArray((1,), np.float64) if want_err else None
    _lib.call("enq_quantize_tensor", code, d_w.ptr, outer, channels, inner, bits,
              _scheme_code(scheme), d_fake.ptr, d_codes.ptr if d_codes else null(), d_s.ptr,
              d_z.ptr, d_err.ptr if d_err else null())
    fake = d_fake.numpy()
    if sshape:
        probe = np.ones(sshape, w.dtype)
    else:
        probe = w.dtype.type(1)     # np.min / np.max of the whole tensor give scalars
    s_like, z_like = _scale_like(probe, probe, bits, scheme)
    scale = _as_container(d_s.numpy().reshape(sshape).astype(np.result_type(s_like),
                                                              copy=False), s_like)
    zp = _as_container(d_z.numpy().reshape(sshape).astype(np.result_type(z_like), copy=False),
                       z_like)
    err_sum = float(d_err.numpy()[0]) if d_err else None
    return fake, scale, zp, d_codes, d_s, err_sum


def quantize_tensor(w: Any, bits: int = 8, scheme: str = "symmetric",
                    per_channel: bool = False, axis: int = 0) -> Tuple[Any, Any, Any]:
    """Fake-quantize one tensor.  Returns ``(quantized, scale, zero_point)``.

    Replaces ``compression/quantization.py:76-93``: per-channel statistics,
    scale, zero point and the fake-quantized tensor come from one fused
    ``enq_quantize_tensor`` call (a single HBM pass for per-channel along
    axis 0)."""
    w = np.asarray(w)
    quant_range(bits, scheme)
    if w.size == 0:
        raise ValueError("zero-size array to reduction operation minimum which has no identity")
    fake, scale, zp, _, _, _ = _quantize_tensor_device(w, bits, scheme, per_channel, axis,
                                                       want_codes=False, want_err=False)
    return fake, scale, zp


#: ``compression/quantization.py:99-112``: which parameters of each layer type
#: are quantized.
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
    """Post-training quantization of a model's weights, in place.

    Replaces ``compression/quantization.py:115-153`` with the same traversal,
    in-place writes, ``quant`` specs and report.  Each tensor is quantized by
    one ``enq_quantize_tensor`` call, which also returns the |error| sum for
    ``mean_abs_error``.  Symmetric tensors of <= 8 bits additionally keep
    their int8 codes and scales on the device (``layer["_state_enq_int8"]``,
    never saved because ``_state_`` keys are excluded by ``Save``), so a later
    ``Forward`` runs the integer kernels without re-deriving them."""
    from ..nn.weights import Int8Weights, store_int8

    report: Dict[str, Any] = {"bits": bits, "scheme": scheme,
                              "per_channel": per_channel, "layers": {}}
    total_err, total_n, float_bytes, int_bits = 0.0, 0, 0, 0
    for i, layer in enumerate(model.layers):
        if layer_types is not None and layer["type"] not in layer_types:
            continue
        for name in QUANTIZABLE.get(layer["type"], ()):
            if name not in layer:
                continue
            original = layer[name]
            src = np.asarray(original)
            quant_range(bits, scheme)
            if src.size == 0:
                raise ValueError(
                    "zero-size array to reduction operation minimum which has no identity")
            keep = (scheme == "symmetric" and bits <= 8 and src.ndim >= 2
                    and src.dtype == np.float32)
            q, scale, zp, d_codes, d_scale, err_sum = _quantize_tensor_device(
                src, bits, scheme, per_channel, 0, want_codes=keep, want_err=True)
            err = float(err_sum / src.size)
            layer[name] = q
            layer.setdefault("quant", {})[name] = {
                "bits": bits, "scheme": scheme,
                "scale": scale, "zero_point": zp}
            if keep:
                store_int8(layer, name, Int8Weights.from_device(q, scale, d_codes, d_scale,
                                                               per_channel, bits))
            report["layers"][f"{i}.{name}"] = {
                "mean_abs_error": err, "size": int(original.size)}
            total_err += err * original.size
            total_n += int(original.size)
            float_bytes += int(original.size) * original.dtype.itemsize
            int_bits += int(original.size) * bits
    report["mean_abs_error"] = total_err / total_n if total_n else 0.0
    report["parameters"] = total_n
    report["float_bytes"] = float_bytes
    report["quantized_bytes"] = int_bits // 8
    report["compression"] = (float_bytes / (int_bits / 8)) if int_bits else 1.0
    return report


class ActivationCalibrator:
    """Records each layer's activation range and installs ``act_quant``
    specs.  Same contract as ``compression/quantization.py:156-209``; the
    model's ``Forward`` is the GPU one when the model runs on enilnets_amd,
    and the per-layer min / max come from ``enq_minmax``."""

    def __init__(self, model: Any, bits: int = 8, scheme: str = "asymmetric",
                 percentile: Optional[float] = None) -> None:
        self.model = model
        self.bits, self.scheme = bits, scheme
        self.percentile = percentile
        self.ranges: Dict[int, List[float]] = {}

    def observe(self, X: Any) -> None:
        """Run one calibration batch and widen the recorded ranges."""
        self.model.Forward(X, training=False)
        for i in range(len(self.model.layers)):
            out = self.model.outputs[i + 1]
            if not hasattr(out, "dtype") or out.dtype.kind != "f":
                continue
            if self.percentile is None:
                low, high = _global_range(out)
            else:
                p = self.percentile
                low, high = _percentiles(out, (100.0 - p, p))
            if i in self.ranges:
                self.ranges[i] = [min(self.ranges[i][0], low), max(self.ranges[i][1], high)]
            else:
                self.ranges[i] = [low, high]

    def apply(self) -> Dict[int, Dict[str, Any]]:
        """Install the observed ranges so ``Forward`` fake-quantizes each
        layer's output.  Returns what was installed."""
        if not self.ranges:
            raise RuntimeError("no calibration data observed -- call observe(X) first")
        installed = {}
        for i, (low, high) in self.ranges.items():
            scale, zero_point = compute_scale(np.asarray(low), np.asarray(high), self.bits,
                                              self.scheme)
            spec = {"bits": self.bits, "scheme": self.scheme,
                    "scale": scale, "zero_point": zero_point,
                    "low": low, "high": high}
            self.model.layers[i]["act_quant"] = spec
            installed[i] = spec
        return installed


def _global_range(x: np.ndarray) -> Tuple[float, float]:
    a = np.ascontiguousarray(x)
    code = _compute_code(a.dtype)
    d_x = DeviceArray.from_numpy(a)
    d_lo, d_hi = DeviceArray((1,), a.dtype), DeviceArray((1,), a.dtype)
    _lib.call("enq_minmax", code, d_x.ptr, 1, 1, a.size, d_lo.ptr, d_hi.ptr)
    return float(d_lo.numpy()[0]), float(d_hi.numpy()[0])


def _percentiles(x: np.ndarray, qs: Sequence[float]) -> List[float]:
    """``float(np.percentile(x, q))`` for each q (NumPy's default 'linear'
    method), as the calibrator's ``quantization.py:186-187`` takes them.

    The order statistics come from ``enq_order_stats`` (a device radix
    select); around them this follows NumPy 2's ``_quantile``: q / 100 and
    the virtual index ``(n - 1) * q`` in the array's float type, the two
    neighbouring ranks (both the last one past the end), and the two-sided
    interpolation of ``_lerp`` (``a + d * t``, or ``b - d * (1 - t)`` for
    ``t >= 0.5``) in that type; a NaN anywhere gives NaN."""
    a = np.ascontiguousarray(x).reshape(-1)
    if a.dtype not in (np.float32, np.float64):
        raise NotImplementedError(f"percentile calibration takes float32 or float64, got {a.dtype}")
    n = a.size
    if n == 0:
        raise IndexError("index -1 is out of bounds for axis 0 with size 0")
    t = a.dtype.type
    plans = []
    for q in qs:
        frac = np.asanyarray(np.true_divide(q, t(100)))
        if not 0.0 <= frac <= 1.0:
            raise ValueError("Percentiles must be in the range [0, 100]")
        vi = np.asanyarray((n - 1) * frac)
        # NumPy's indexes: -1 (the last element) for both at or past the end,
        # and gamma taken against that -1
        if vi >= n - 1:
            lo_i = hi_i = -1
        elif vi < 0:
            lo_i = hi_i = 0
        else:
            lo_i = int(np.floor(vi))
            hi_i = lo_i + 1
        gamma = np.asanyarray(vi - np.intp(lo_i), dtype=vi.dtype)
        plans.append((lo_i % n, hi_i % n, gamma))
    ranks = sorted({r for lo_i, hi_i, _ in plans for r in (lo_i, hi_i)} | {n - 1})
    d_x = DeviceArray.from_numpy(a)
    d_out = DeviceArray((len(ranks),), a.dtype)
    host_ranks = (ctypes.c_int64 * len(ranks))(*ranks)
    _lib.call("enq_order_stats", _compute_code(a.dtype), d_x.ptr, n, host_ranks, len(ranks),
              d_out.ptr)
    vals = dict(zip(ranks, d_out.numpy()))
    if np.isnan(vals[n - 1]):           # NaN sorts last: any NaN makes every result NaN
        return [float("nan")] * len(plans)
    result = []
    for lo_i, hi_i, gamma in plans:
        lo, hi = np.asanyarray(vals[lo_i]), np.asanyarray(vals[hi_i])
        diff = np.subtract(hi, lo)
        v = np.asanyarray(np.add(lo, diff * gamma))
        if gamma >= 0.5:
            v = np.asanyarray(np.subtract(hi, diff * (1 - gamma)), dtype=v.dtype)
        result.append(float(v))
    return result


def remove_activation_quantization(model: Any) -> None:
    """Drop every activation-quantization spec (``quantization.py:212-215``)."""
    for layer in model.layers:
        layer.pop("act_quant", None)


def quantization_error(reference: Sequence[Any], candidate: Sequence[Any]) -> Dict[str, float]:
    """Compare two sets of model outputs.

    Replaces ``compression/quantization.py:218-229``; the four sums come from
    ``enq_error_stats`` (accumulated in float64)."""
    a = np.concatenate([np.asarray(v).reshape(-1) for v in reference])
    b = np.concatenate([np.asarray(v).reshape(-1) for v in candidate])
    if a.shape != b.shape:
        raise ValueError(f"operands could not be broadcast together with shapes {a.shape} {b.shape}")
    dtype = np.result_type(_probe(b) - _probe(a))
    code = _compute_code(dtype)
    if a.size == 0:
        raise ValueError("zero-size array to reduction operation maximum which has no identity")
    d_a = DeviceArray.from_numpy(np.ascontiguousarray(a, dtype=dtype))
    d_b = DeviceArray.from_numpy(np.ascontiguousarray(b, dtype=dtype))
    out = (ctypes.c_double * 4)()
    _lib.call("enq_error_stats", code, d_a.ptr, d_b.ptr, a.size, out)
    sum_abs, max_abs, sum_aa, sum_dd = out[0], out[1], out[2], out[3]
    denom = float(np.sqrt(sum_aa))
    return {"mean_abs_error": float(sum_abs / a.size),
            "max_abs_error": float(max_abs),
            "relative_error": float(np.sqrt(sum_dd) / denom) if denom > 0 else 0.0}
