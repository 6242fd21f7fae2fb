"""Dense layers on int8 weights, device-resident.

``dense_w8`` is the fp32-activation path (``Enilnets/nn/forward.py:317-321``
with the fake-quantized weights); ``dense_w8a8`` the integer path with
per-token activation codes.  Inputs and outputs are ``DeviceArray``s, so a
model's layers chain in HBM without host round trips.
"""

from typing import Any, Dict, Optional, Tuple

import numpy as np

from .. import _lib
from ..device import DeviceArray, null
from .weights import Int8Weights

VARIANTS = {"fp32": _lib.W8_FP32, "bf16": _lib.W8_BF16}

#: ``Enilnets/core/constants.py:18,21,22``.
SIGMOID_CLIP = 500.0
LEAKYRELU_ALPHA = 0.01
ELU_ALPHA = 1.0


def activation_args(name: str, params: Optional[Dict[str, Any]] = None) -> Tuple[int, float, float]:
    """(code, alpha, clip) of an activation (``nn/activations.py:6-42``);
    ValueError for an unknown name, as ``activate`` raises."""
    if name not in _lib.ACTIVATIONS:
        raise ValueError(f"Unknown activation: {name!r}")
    params = params or {}
    alpha = params.get("alpha")
    if alpha is None:
        alpha = ELU_ALPHA if name == "elu" else LEAKYRELU_ALPHA
    clip = params.get("sigmoid_clip")
    if clip is None:
        clip = SIGMOID_CLIP
    return _lib.ACTIVATIONS[name], float(alpha), float(clip)


def _promotion_key(v: Any) -> Tuple[Any, ...]:
    """What NumPy's promotion of ``v`` depends on: arrays and NumPy scalars by
    dtype, Python scalars (weak) by type."""
    if isinstance(v, (np.ndarray, np.generic)):
        return (isinstance(v, np.ndarray), v.dtype.str)
    return (type(v),)


# result dtype of ``x / scale + zero_point`` by promotion keys and the
# output dtype: the spec is applied per layer call, and resolving it on
# probe values each time cost more host time than the device pass
_AQ_RESULT: Dict[Tuple[Any, ...], Any] = {}


def act_quant_args(spec: Dict[str, Any], out_dtype: Any = np.float32) -> Tuple[Any, ...]:
    """``(mode, scale, zero_point, qmin, qmax, result_dtype)`` of an
    ``act_quant`` spec (``forward.py:798-805``) applied to a layer output of
    host dtype ``out_dtype``.  The arithmetic is the dtype NumPy gives
    ``x / scale + zero_point`` (the calibrator's float64 0-d scale makes it
    float64 even for float32 outputs)."""
    from ..compression.quantization import _probe, quant_range
    qmin, qmax = quant_range(spec["bits"], spec["scheme"])
    scale, zp = spec["scale"], spec["zero_point"]
    if np.size(scale) != 1 or np.size(zp) != 1:
        raise NotImplementedError("act_quant specs are per tensor on the quantized path")
    key = (_promotion_key(scale), _promotion_key(zp), np.dtype(out_dtype).str)
    res = _AQ_RESULT.get(key)
    if res is None:
        res = (np.ones(1, dtype=out_dtype) / _probe(scale) + _probe(zp)).dtype
        _AQ_RESULT[key] = res
    if res not in (np.float32, np.float64):
        raise NotImplementedError(f"act_quant arithmetic in {res} is not supported")
    mode = _lib.AQ_F64 if res == np.float64 else _lib.AQ_F32
    return (mode, float(np.asarray(scale).reshape(-1)[0]), float(np.asarray(zp).reshape(-1)[0]),
            float(qmin), float(qmax), res)


def act_quant(x: DeviceArray, spec: Dict[str, Any], out_dtype: Any = np.float32,
              out: Optional[DeviceArray] = None) -> DeviceArray:
    """The standalone fake-quantization pass of a layer output."""
    mode, scale, zp, qmin, qmax, _ = act_quant_args(spec, out_dtype)
    y = out if out is not None else DeviceArray(x.shape, np.float32)
    _lib.call("enq_act_quant", x.ptr, x.size, mode, scale, zp, qmin, qmax, y.ptr)
    return y


def _rows(x: DeviceArray) -> Tuple[int, int]:
    k = x.shape[-1]
    return x.size // max(k, 1), k


def dense_w8(x: DeviceArray, w: Int8Weights, bias: Optional[DeviceArray] = None,
             activation: str = "linear", activation_params: Optional[Dict[str, Any]] = None,
             variant: str = "fp32", out: Optional[DeviceArray] = None,
             pre_activation: Optional[DeviceArray] = None,
             act_quant: Optional[Dict[str, Any]] = None,
             out_dtype: Any = np.float32) -> DeviceArray:
    """``act(x @ (codes * scale).T + bias)`` for fp32 ``x`` of shape
    ``(..., k)`` and int8 weights ``(n, k)``.  ``act_quant`` (a layer's
    calibrated spec) fake-quantizes the output in the same epilogue, in the
    arithmetic NumPy uses for an output of host dtype ``out_dtype``."""
    if x.dtype != np.float32:
        raise NotImplementedError(f"W8 Dense takes float32 activations, got {x.dtype}")
    m, k = _rows(x)
    n, wk = w.shape[-2], w.shape[-1]
    if len(w.shape) != 2:
        raise ValueError(f"dense weights must be 2-D, got shape {w.shape}")
    if wk != k:
        raise ValueError(f"shapes {x.shape} and {w.shape} not aligned: {k} (dim -1) != {wk}")
    code, alpha, clip = activation_args(activation, activation_params)
    out_shape = x.shape[:-1] + (n,)
    y = out if out is not None else DeviceArray(out_shape, np.float32)
    z = pre_activation.ptr if pre_activation is not None else null()
    b = bias.ptr if bias is not None else null()
    if act_quant is None:
        _lib.call("enq_dense_w8", x.ptr, m, k, w.codes.ptr, w.scale.ptr, n, b, code, alpha, clip,
                  VARIANTS[variant], y.ptr, z)
    else:
        mode, scale, zp, qmin, qmax, _ = act_quant_args(act_quant, out_dtype)
        _lib.call("enq_dense_w8_aq", x.ptr, m, k, w.codes.ptr, w.scale.ptr, n, b, code, alpha,
                  clip, VARIANTS[variant], mode, scale, zp, qmin, qmax, y.ptr, z)
    return y


def dense_w8_ffn(x: DeviceArray, w1: Int8Weights, b1: Optional[DeviceArray], act1: str,
                 w2: Int8Weights, b2: Optional[DeviceArray] = None, act2: str = "linear",
                 variant: str = "fp32", out: Optional[DeviceArray] = None,
                 params1: Optional[Dict[str, Any]] = None,
                 params2: Optional[Dict[str, Any]] = None,
                 bound: Optional[DeviceArray] = None) -> DeviceArray:
    """Two Dense layers in a row, ``act2(act1(x W1^T + b1) W2^T + b2)``, when
    only the second output is wanted (a transformer block's feed-forward
    pair): ``dense_w8`` twice, except that at large sizes the first GEMM
    writes its output straight as the second's fp16/e4m3 split.  ``bound``
    is ``ffn_bound(w1, b1, act1, params1)``, computed once per weight (None:
    computed in every call)."""
    if x.dtype != np.float32:
        raise NotImplementedError(f"W8 Dense takes float32 activations, got {x.dtype}")
    m, k = _rows(x)
    if len(w1.shape) != 2 or len(w2.shape) != 2:
        raise ValueError("dense weights must be 2-D")
    n1, n2 = w1.shape[0], w2.shape[0]
    if w1.shape[1] != k or w2.shape[1] != n1:
        raise ValueError(f"shapes {x.shape}, {w1.shape} and {w2.shape} not aligned")
    c1, a1, k1 = activation_args(act1, params1)
    c2, a2, k2 = activation_args(act2, params2)
    y = out if out is not None else DeviceArray(x.shape[:-1] + (n2,), np.float32)
    _lib.call("enq_dense_w8_ffn", x.ptr, m, k, w1.codes.ptr, w1.scale.ptr, n1,
              b1.ptr if b1 is not None else null(), c1, a1, k1,
              bound.ptr if bound is not None else null(), w2.codes.ptr, w2.scale.ptr, n2,
              b2.ptr if b2 is not None else null(), c2, a2, k2, VARIANTS[variant], y.ptr)
    return y


def ffn_bound(w: Int8Weights, bias: Optional[DeviceArray], activation: str,
              activation_params: Optional[Dict[str, Any]] = None) -> DeviceArray:
    """The output bound of a Dense layer that ``dense_w8_ffn`` uses for its
    hidden rows' exponents (two floats on the device): a property of the
    weights, bias and activation only."""
    n, k = w.shape[-2], w.shape[-1]
    code, alpha, clip = activation_args(activation, activation_params)
    out = DeviceArray((2,), np.float32)
    _lib.call("enq_f16f8_bound", w.codes.ptr, n, k, w.scale.ptr,
              bias.ptr if bias is not None else null(), code, alpha, clip, out.ptr)
    return out


class ActivationPlanes:
    """Activations split once into the bf16 planes the tile kernels read
    (``split_planes``), for several ``dense_w8_planes`` calls."""

    def __init__(self, data: DeviceArray, shape: Tuple[int, ...], variant: str):
        self.data, self.shape, self.variant = data, shape, variant


def split_planes(x: DeviceArray, variant: str = "fp32") -> ActivationPlanes:
    """bf16 planes of fp32 ``x`` (``..., k``): hi = bf16(x) and, for the
    fp32-accurate variant, lo = bf16(x - hi); rows padded to a multiple of 32."""
    if x.dtype != np.float32:
        raise NotImplementedError(f"W8 Dense takes float32 activations, got {x.dtype}")
    m, k = _rows(x)
    kp = -(-k // 32) * 32
    planes = DeviceArray((2 if variant == "fp32" else 1, m, kp), np.uint16)
    _lib.call("enq_split_planes", x.ptr, m, k, VARIANTS[variant], planes.ptr)
    return ActivationPlanes(planes, x.shape, variant)


def dense_w8_planes(xp: ActivationPlanes, w: Int8Weights, bias: Optional[DeviceArray] = None,
                    activation: str = "linear",
                    activation_params: Optional[Dict[str, Any]] = None,
                    out: Optional[DeviceArray] = None,
                    pre_activation: Optional[DeviceArray] = None) -> DeviceArray:
    """``dense_w8`` on activations already split by ``split_planes`` (the
    tile kernels of ``dense_w8``, without the split)."""
    k = xp.shape[-1]
    m = int(np.prod(xp.shape[:-1], dtype=np.int64))
    n, wk = w.shape[-2], w.shape[-1]
    if len(w.shape) != 2:
        raise ValueError(f"dense weights must be 2-D, got shape {w.shape}")
    if wk != k:
        raise ValueError(f"shapes {xp.shape} and {w.shape} not aligned: {k} (dim -1) != {wk}")
    code, alpha, clip = activation_args(activation, activation_params)
    y = out if out is not None else DeviceArray(xp.shape[:-1] + (n,), np.float32)
    z = pre_activation.ptr if pre_activation is not None else null()
    b = bias.ptr if bias is not None else null()
    _lib.call("enq_gemm_w8_planes", xp.data.ptr, m, k, w.codes.ptr, w.scale.ptr, n, b, code,
              alpha, clip, VARIANTS[xp.variant], y.ptr, z)
    return y


class SplitActivations:
    """Activations split once for the large-tile fp32-accurate GEMM
    (``split_f16f8``): fp16 high parts, e4m3 low parts and a power-of-two
    exponent per row, for several ``dense_w8_split`` calls."""

    def __init__(self, data: DeviceArray, shape: Tuple[int, ...]):
        self.data, self.shape = data, shape


def split_f16f8(x: DeviceArray) -> SplitActivations:
    """The fp32-accurate split of fp32 ``x`` (``..., k``): per row the power of
    two e with max |x| * 2^e in [2^14, 2^15), hi = fp16(x * 2^e) and
    lo = e4m3(x * 2^e - hi), rows padded to a multiple of 64."""
    if x.dtype != np.float32:
        raise NotImplementedError(f"W8 Dense takes float32 activations, got {x.dtype}")
    m, k = _rows(x)
    kp = -(-k // 64) * 64
    buf = DeviceArray((m * (3 * kp + 4),), np.uint8)
    _lib.call("enq_split_f16f8", x.ptr, m, k, buf.ptr)
    return SplitActivations(buf, x.shape)


def dense_w8_split(xs: SplitActivations, w: Int8Weights, bias: Optional[DeviceArray] = None,
                   activation: str = "linear",
                   activation_params: Optional[Dict[str, Any]] = None,
                   out: Optional[DeviceArray] = None,
                   pre_activation: Optional[DeviceArray] = None) -> DeviceArray:
    """``dense_w8`` (fp32-accurate) on activations already split by
    ``split_f16f8``: the large-tile GEMM of ``dense_w8`` without the split.
    Needs K a multiple of 16."""
    k = xs.shape[-1]
    m = int(np.prod(xs.shape[:-1], dtype=np.int64))
    n, wk = w.shape[-2], w.shape[-1]
    if len(w.shape) != 2:
        raise ValueError(f"dense weights must be 2-D, got shape {w.shape}")
    if wk != k:
        raise ValueError(f"shapes {xs.shape} and {w.shape} not aligned: {k} (dim -1) != {wk}")
    code, alpha, clip = activation_args(activation, activation_params)
    y = out if out is not None else DeviceArray(xs.shape[:-1] + (n,), np.float32)
    z = pre_activation.ptr if pre_activation is not None else null()
    b = bias.ptr if bias is not None else null()
    _lib.call("enq_gemm_w8_f16f8", xs.data.ptr, m, k, w.codes.ptr, w.scale.ptr, n, b, code,
              alpha, clip, y.ptr, z)
    return y


def dense_w8a8(x: DeviceArray, w: Int8Weights, bias: Optional[DeviceArray] = None,
               activation: str = "linear", activation_params: Optional[Dict[str, Any]] = None,
               out: Optional[DeviceArray] = None,
               acc: Optional[DeviceArray] = None,
               x_spec: Optional[Dict[str, Any]] = None,
               x_dtype: Any = np.float32) -> DeviceArray:
    """int8 activation codes times int8 weights, int32 accumulation (``acc``
    receives the accumulators when given).  The activations are quantized
    per token (symmetric, dynamic), or with ``x_spec`` -- the calibrated
    ``act_quant`` spec of the layer that produced ``x``, whose host dtype is
    ``x_dtype`` -- per tensor on that spec's grid (static W8A8)."""
    if x.dtype != np.float32:
        raise NotImplementedError(f"W8A8 Dense takes float32 activations, got {x.dtype}")
    m, k = _rows(x)
    n, wk = w.shape[-2], w.shape[-1]
    if wk != k:
        raise ValueError(f"shapes {x.shape} and {w.shape} not aligned: {k} (dim -1) != {wk}")
    code, alpha, clip = activation_args(activation, activation_params)
    y = out if out is not None else DeviceArray(x.shape[:-1] + (n,), np.float32)
    b = bias.ptr if bias is not None else null()
    a = acc.ptr if acc is not None else null()
    if x_spec is None:
        _lib.call("enq_dense_w8a8", x.ptr, m, k, w.codes.ptr, w.scale.ptr, n, b, code, alpha,
                  clip, y.ptr, a)
        return y
    mode, scale, zp, qmin, qmax, _ = act_quant_args(x_spec, x_dtype)
    # the zero-point term needs the weight's code sums unless it vanishes
    shift = 128 if qmax > 127 else 0
    sums = w.code_sums.ptr if shift != zp else null()
    _lib.call("enq_dense_w8a8_static", x.ptr, m, k, mode, scale, zp, qmin, qmax, w.codes.ptr,
              w.scale.ptr, sums, n, b, code, alpha, clip, y.ptr, a)
    return y


def quantize_rows_i8(x: DeviceArray) -> Tuple[DeviceArray, DeviceArray]:
    """Per-row (per-token) symmetric int8 codes and fp32 scales."""
    m, k = _rows(x)
    codes = DeviceArray(x.shape, np.int8)
    scale = DeviceArray((m,), np.float32)
    _lib.call("enq_quantize_rows_i8", x.ptr, m, k, codes.ptr, scale.ptr)
    return codes, scale


def gemm_w8a8(x_codes: DeviceArray, x_scale: DeviceArray, w: Int8Weights,
              bias: Optional[DeviceArray] = None, activation: str = "linear",
              out: Optional[DeviceArray] = None,
              acc: Optional[DeviceArray] = None) -> DeviceArray:
    """The integer GEMM on already-quantized activations."""
    m, k = _rows(x_codes)
    n = w.shape[-2]
    code, alpha, clip = activation_args(activation)
    y = out if out is not None else DeviceArray(x_codes.shape[:-1] + (n,), np.float32)
    _lib.call("enq_gemm_w8a8", x_codes.ptr, x_scale.ptr, w.codes.ptr, w.scale.ptr,
              bias.ptr if bias is not None else null(), m, n, k, code, alpha, clip, y.ptr,
              acc.ptr if acc is not None else null())
    return y


def quantize_weight_rows(w: np.ndarray) -> Int8Weights:
    """Per-output-channel symmetric int8 codes of a float32 ``(n, k)`` weight
    on the device (``quantize_tensor(w, 8, per_channel=True)`` semantics)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError(f"expected a 2-D weight, got shape {w.shape}")
    d_w = DeviceArray.from_numpy(w)
    codes, scale = quantize_rows_i8(d_w)
    return Int8Weights(codes, scale, w.shape, 8, True, None, None)
