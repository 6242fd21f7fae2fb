"""Device-resident mixture-of-experts layer (``Enilnets/nn/moe.py:52-87``).

The router, the routing, both expert GEMMs and the gated combine run in one
library call (``enq_moe_w8``) on the layer's int8 ``Wr``, ``W1`` and ``W2``
codes; group sizes never leave the device.  The load-balancing loss the
reference stores in ``layer["_state_aux_loss"]`` (``moe.py:67-68``) is
computed on the device as well.
"""

from typing import Any, Dict, Optional, Tuple

import numpy as np

from .. import _lib
from ..device import DeviceArray, null
from .dense import VARIANTS, activation_args
from .weights import Int8Weights, int8_weights


def _stacked_bias(layer: Dict[str, Any], key: str, shape: Tuple[int, int]) -> Optional[DeviceArray]:
    b = layer.get(key)
    if b is None:
        return None
    b = np.ascontiguousarray(b, dtype=np.float32)
    if b.size != shape[0] * shape[1]:
        raise ValueError(f"{key} of shape {b.shape} does not match {shape}")
    return DeviceArray.from_numpy(b.reshape(-1))


def moe_biases(layer: Dict[str, Any]) -> Tuple[Optional[DeviceArray], ...]:
    """``(b1, b2, br)`` of the layer as float32 device vectors (None where
    the layer has none)."""
    n_exp, d = int(layer["num_experts"]), int(layer["embed_dim"])
    hidden = np.shape(layer["W1"])[1]
    br = layer.get("br")
    return (_stacked_bias(layer, "b1", (n_exp, hidden)), _stacked_bias(layer, "b2", (n_exp, d)),
            DeviceArray.from_numpy(np.ascontiguousarray(br, dtype=np.float32).reshape(-1))
            if br is not None else None)


def moe_forward(x: DeviceArray, layer: Dict[str, Any], variant: str = "fp32",
                router_logits: Optional[DeviceArray] = None,
                want_routing: bool = False, out: Optional[DeviceArray] = None,
                biases: Optional[Tuple[Optional[DeviceArray], ...]] = None,
                aux_loss: bool = True,
                weights: Optional[Tuple[Int8Weights, Int8Weights, Optional[Int8Weights]]] = None,
                bound: Optional[DeviceArray] = None
                ) -> Tuple[DeviceArray, Dict[str, Any]]:
    """``(out, info)`` for a ``(..., E)`` float32 device array.  ``info``
    holds ``aux_loss`` (a Python float, unless ``aux_loss`` is False) and,
    with ``want_routing``, the device arrays ``probs`` (tokens, experts) and
    ``top_idx`` (tokens, k).  ``router_logits`` replaces the router GEMM (the
    benchmark configuration draws the logits directly); ``biases`` passes
    ``moe_biases(layer)`` made once and ``weights`` the ``(W1, W2, Wr)``
    int8 weights, skipping the per-call staleness check of the layer's
    cache (which hashes the host arrays); ``bound`` passes ``moe_bound`` of
    those weights, computed once."""
    if x.dtype != np.float32:
        raise NotImplementedError(f"the MoE layer takes float32 activations, got {x.dtype}")
    if layer["activation"] == "softmax":
        raise NotImplementedError("softmax expert activations are not on the quantized path")
    d = int(layer["embed_dim"])
    n_exp = int(layer["num_experts"])
    k = int(layer["top_k"])
    if x.shape[-1] != d:
        raise ValueError(f"input width {x.shape[-1]} does not match embed_dim {d}")
    tokens = x.size // d
    if weights is None:
        weights = (int8_weights(layer, "W1"), int8_weights(layer, "W2"),
                   int8_weights(layer, "Wr") if router_logits is None else None)
    w1, w2, wr = weights
    if len(w1.shape) != 3 or len(w2.shape) != 3:
        raise ValueError("W1 and W2 must be stacked (experts, rows, cols) weights")
    hidden = w1.shape[1]
    if w1.shape != (n_exp, hidden, d) or w2.shape != (n_exp, d, hidden):
        raise ValueError(f"expert weights {w1.shape} / {w2.shape} do not match "
                         f"({n_exp}, hidden, {d})")
    code, alpha, clip = activation_args(layer["activation"], layer.get("activation_params"))
    b1, b2, d_br = moe_biases(layer) if biases is None else biases
    if router_logits is None:
        if wr is None:
            raise ValueError("router weights are needed when no router logits are given")
        if wr.shape != (n_exp, d):
            raise ValueError(f"router weights {wr.shape} do not match ({n_exp}, {d})")
        router = (null(), wr.codes.ptr, wr.scale.ptr, d_br.ptr if d_br is not None else null())
    else:
        if router_logits.shape[-1] != n_exp or router_logits.size != tokens * n_exp:
            raise ValueError(f"router logits {router_logits.shape} do not match "
                             f"({tokens}, {n_exp})")
        router = (router_logits.ptr, null(), null(), null())
    out = out if out is not None else DeviceArray(x.shape, np.float32)
    probs = DeviceArray((tokens, n_exp), np.float32) if want_routing else None
    top_idx = DeviceArray((tokens, k), np.int32) if want_routing else None
    loss = DeviceArray((1,), np.float64) if aux_loss else None
    _lib.call("enq_moe_w8", x.ptr, tokens, d, *router, w1.codes.ptr, w1.scale.ptr,
              b1.ptr if b1 is not None else null(), w2.codes.ptr, w2.scale.ptr,
              b2.ptr if b2 is not None else null(), n_exp, hidden, k, code, alpha, clip,
              bound.ptr if bound is not None else null(), VARIANTS[variant], out.ptr, probs.ptr if probs is not None else null(),
              top_idx.ptr if top_idx is not None else null(),
              loss.ptr if loss is not None else null())
    info: Dict[str, Any] = {}
    if loss is not None:
        info["aux_loss"] = float(loss.numpy()[0])
    if want_routing:
        info["probs"] = probs
        info["top_idx"] = top_idx
    return out, info


def moe_bound(layer: Dict[str, Any], w1: Int8Weights,
              b1: Optional[DeviceArray]) -> DeviceArray:
    """The first expert layer's output bound (two floats on the device) that
    the fp16/e4m3 path of ``moe_forward`` uses for the hidden rows'
    exponents: ``enq_f16f8_bound`` over the stacked (experts * hidden, d)
    codes, scales and biases under the layer's activation.  A property of
    the weights only."""
    rows, k = w1.shape[0] * w1.shape[1], w1.shape[2]
    code, alpha, clip = activation_args(layer["activation"], layer.get("activation_params"))
    out = DeviceArray((2,), np.float32)
    _lib.call("enq_f16f8_bound", w1.codes.ptr, rows, k, w1.scale.ptr,
              b1.ptr if b1 is not None else null(), code, alpha, clip, out.ptr)
    return out
