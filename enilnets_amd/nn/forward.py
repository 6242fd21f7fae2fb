"""Drop-in ``Forward`` for quantized models on MI355X.

Mirrors ``Enilnets/nn/forward.py:272-811`` for the layer types of the
quantized-inference path: the input is cast to float32 (the reference's
default working dtype, ``:285``), every layer runs on the device, and
``model.outputs`` / ``model.pre_activations`` are filled with host arrays as
the reference fills them (``:295-302,810``).  Dense, attention-projection
and expert weights run on their int8 codes (``enilnets_amd.nn.weights``).
Layer types outside this path raise NotImplementedError instead of silently
computing on the host.
"""

from typing import Any, Dict, List, Optional

import numpy as np

from ..device import DeviceArray
from .dense import act_quant, act_quant_args, dense_w8
from .moe import moe_forward
from .transformer import (embedding, layernorm, mha_forward, positional_encoding,
                          residual_add)
from .weights import int8_weights

#: Activations whose NumPy result is float64 for a float32 input, because
#: ``activations.py:32`` multiplies by ``np.sqrt(2 / np.pi)`` (a float64
#: NumPy scalar) and NumPy 2 promotes the result.
_FLOAT64_ACTIVATIONS = {"gelu"}


def _bias(layer: Dict[str, Any], key: str, n: int) -> DeviceArray:
    b = layer.get(key)
    if b is None:
        b = np.zeros(n, np.float32)
    return DeviceArray.from_numpy(np.ascontiguousarray(b, dtype=np.float32))


def _dense(cur: DeviceArray, layer: Dict[str, Any], variant: str):
    """Dense layer; a calibrated ``act_quant`` runs in the GEMM epilogue."""
    w = int8_weights(layer, "weights")
    n = w.shape[0]
    z = DeviceArray(cur.shape[:-1] + (n,), np.float32)
    dtype = np.float64 if layer["activation"] in _FLOAT64_ACTIVATIONS else np.float32
    y = dense_w8(cur, w, _bias(layer, "bias", n), layer["activation"],
                 layer.get("activation_params", {}), variant, pre_activation=z,
                 act_quant=layer.get("act_quant"), out_dtype=dtype)
    return y, z, dtype


def Forward(model: Any, inputs: Any, training: bool = False, dropout_rate: float = 0.0,
            variant: str = "fp32") -> np.ndarray:
    """Run ``inputs`` through ``model.layers`` on the GPU.  Returns the last
    layer's output and fills ``model.outputs`` and ``model.pre_activations``
    like the reference.  ``variant`` selects the W8 Dense arithmetic
    ("fp32": fp32-accurate, "bf16": bf16 activations).

    Layer types: dense/sparse, layernorm, multihead_attention (softmax),
    residual_save, residual_add, moe, embedding, positional_encoding and
    dropout (inference).  Every layer computes in float32 on
    the device; the host copy of each output takes the dtype NumPy gives the
    reference's expression (float64 after GELU, ``forward.py:32``; after
    attention, whose scores are divided by the float64 ``np.sqrt(Dh)``,
    ``:525``; and wherever a float64 operand propagates)."""
    x = np.asarray(inputs, dtype=np.float32)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    outputs: List[np.ndarray] = [x]
    pre: List[Optional[np.ndarray]] = [None]
    dev: List[DeviceArray] = [DeviceArray.from_numpy(x)]
    for layer in model.layers:
        cur = dev[-1]
        cur_dtype = outputs[-1].dtype
        kind = layer["type"]
        z_host = None
        if kind in ("dense", "sparse"):
            y, z, dtype = _dense(cur, layer, variant)
            z_host = z.numpy()
        elif kind == "layernorm":
            y = layernorm(cur, layer)
            dtype = np.result_type(cur_dtype, np.asarray(layer["gamma"]).dtype,
                                   np.asarray(layer["beta"]).dtype)
        elif kind == "multihead_attention":
            y = mha_forward(cur, layer, variant, training)
            dtype = np.float64
        elif kind == "residual_save":
            y, dtype = cur, cur_dtype
        elif kind == "embedding":
            # indices come from the host input, as forward.py:414-422 reads them
            y = embedding(outputs[-1], layer)
            dtype = np.asarray(layer["weights"]).dtype
        elif kind == "positional_encoding":
            y = positional_encoding(cur, layer)
            key = "weights" if layer.get("_pos_type") == "learnable" else "pe"
            dtype = np.result_type(cur_dtype, np.asarray(layer[key]).dtype)
        elif kind == "dropout":
            rate = layer.get("rate", dropout_rate)
            if training and rate > 0:
                raise NotImplementedError("training-mode dropout is not on the quantized path")
            layer["mask"] = None
            y, dtype = cur, cur_dtype
        elif kind == "residual_add":
            idx = layer["save_index"]
            y = residual_add(cur, dev[idx])
            dtype = np.result_type(cur_dtype, outputs[idx].dtype)
        elif kind == "moe":
            y, info = moe_forward(cur, layer, variant)
            layer["_state_aux_loss"] = info["aux_loss"]
            dtype = cur_dtype
        else:
            raise NotImplementedError(
                f"layer type {kind!r} is not on enilnets_amd's quantized path")
        spec = layer.get("act_quant")
        if spec is not None:
            if kind not in ("dense", "sparse"):  # a Dense epilogue applied it already
                y = act_quant(y, spec, dtype)
            dtype = act_quant_args(spec, dtype)[-1]
        if y is cur:
            host = outputs[-1]
        else:
            host = y.numpy()
            if host.dtype != dtype:
                host = host.astype(dtype)
        dev.append(y)
        outputs.append(host)
        pre.append(z_host)
    model.outputs = outputs
    model.pre_activations = pre
    return outputs[-1]
