"""NumPy restatement of the Enilnets forward pieces the quantized path runs.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): never imported by the
product package.

Covers the Dense branch (``Enilnets/nn/forward.py:316-324``), the elementwise
activations it applies (``Enilnets/nn/activations.py:6-42``), LayerNorm
(``forward.py:207-254``), the softmax multi-head attention branch with its
four projections (``forward.py:423-430,525-551``), residual save/add
(``forward.py:684-689,762-766``), the Mixture-of-Experts layer
(``Enilnets/nn/moe.py:23-87``) and the composed W8A8 Dense the reference does
not have (quantize activations per token with the reference's own
``quantize_tensor``, integer GEMM, rescale).
"""

from typing import Any, Dict, List, Optional, Tuple

import numpy as np

from .quantization import quantize, quantize_tensor

#: ``Enilnets/core/constants.py:18,21,22``.
SIGMOID_CLIP = 500.0
LEAKYRELU_ALPHA = 0.01
ELU_ALPHA = 1.0


def activate(name: str, x: Any, alpha: Optional[float] = None,
             sigmoid_clip: Optional[float] = None) -> Any:
    """Elementwise activation.  Follows ``nn/activations.py:6-42``."""
    clip = SIGMOID_CLIP if sigmoid_clip is None else sigmoid_clip
    if name == "linear":
        return x
    if name == "relu":
        return np.maximum(0, x)
    if name == "leakyrelu":
        a = LEAKYRELU_ALPHA if alpha is None else alpha
        return np.where(x > 0, x, a * x)
    if name == "elu":
        a = ELU_ALPHA if alpha is None else alpha
        return np.where(x > 0, x, a * (np.exp(x) - 1))
    if name == "selu":
        lam = 1.0507009873554804934193349852946
        alp = 1.6732632423543772848170429916717
        return lam * np.where(x > 0, x, alp * (np.exp(x) - 1))
    if name == "gelu":
        inner = np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)
        return 0.5 * x * (1 + np.tanh(inner))
    if name == "swish":
        return x * 1.0 / (1.0 + np.exp(-x))
    if name == "mish":
        return x * np.tanh(np.log(1 + np.exp(x)))
    if name == "sigmoid":
        return 1.0 / (1.0 + np.exp(-np.clip(x, -clip, clip)))
    if name == "tanh":
        return np.tanh(x)
    if name == "softmax":
        shifted = np.exp(x - np.max(x, axis=-1, keepdims=True))
        return shifted / np.sum(shifted, axis=-1, keepdims=True)
    if name == "softplus":
        return np.log(1 + np.exp(np.clip(x, -clip, clip)))
    raise ValueError(f"Unknown activation: {name!r}")


def dense_forward(layer: Dict[str, Any], x: Any,
                  compute_dtype: Any = np.float32) -> Tuple[Any, Any]:
    """``(activated, pre_activation)`` of one dense layer.

    Follows ``nn/forward.py:317-321``: ``z = x @ W.T + b`` in the compute
    dtype, cast back, then the layer's activation."""
    w = layer["weights"]
    z = np.dot(x.astype(compute_dtype), w.astype(compute_dtype).T) + \
        layer["bias"].astype(compute_dtype)
    z = z.astype(compute_dtype)
    out = activate(layer["activation"], z, **layer.get("activation_params", {}))
    return out, z


def layernorm_forward(x: Any, layer: Dict[str, Any]) -> Any:
    """LayerNorm over the last axis of a 2-D or 3-D input.  Follows
    ``nn/forward.py:207-254`` (the 2-D and 3-D branches)."""
    eps = layer.get("epsilon", 1e-5)
    if x.ndim not in (2, 3):
        raise ValueError("oracle layernorm covers 2-D and 3-D inputs only")
    axis = x.ndim - 1
    shape = (1,) * (x.ndim - 1) + (-1,)
    gamma = layer["gamma"].reshape(shape)
    beta = layer["beta"].reshape(shape)
    mu = np.mean(x, axis=axis, keepdims=True)
    var = np.var(x, axis=axis, keepdims=True)
    return gamma * ((x - mu) / np.sqrt(var + eps)) + beta


def window_mask(seq: int, causal: bool, window: Optional[int]) -> Optional[Any]:
    """Additive attention mask, following ``nn/forward.py:102-117``: -inf
    where key j may not be seen from query i (causal: j > i; window:
    |i - j| > window), else 0; None when nothing is masked."""
    if not causal and window is None:
        return None
    pos = np.arange(seq)
    diff = pos[:, None] - pos[None, :]
    blocked = diff < 0 if causal else np.zeros(diff.shape, dtype=bool)
    if window is not None:
        blocked = blocked | (np.abs(diff) > window)
    return np.where(blocked, -np.inf, 0.0)


def mha_forward(x: Any, layer: Dict[str, Any]) -> Any:
    """Softmax multi-head self-attention with absolute positions.

    Follows ``nn/forward.py:423-430`` (projections), ``:525,538-549``
    (scores, causal / sliding-window mask, softmax, context) and ``:550-551``
    (output projection).  Grouped K/V heads are expanded group-major as in
    ``forward.py:165-171``."""
    B, S, E = x.shape
    H = layer["num_heads"]
    Dh = layer["head_dim"]
    Hkv = layer.get("num_kv_heads", H)
    q = np.dot(x, layer["Wq"].T) + layer["bq"]
    k = np.dot(x, layer["Wk"].T) + layer["bk"]
    v = np.dot(x, layer["Wv"].T) + layer["bv"]
    qh = q.reshape(B, S, H, Dh).transpose(0, 2, 1, 3)
    kh = k.reshape(B, S, Hkv, Dh).transpose(0, 2, 1, 3)
    vh = v.reshape(B, S, Hkv, Dh).transpose(0, 2, 1, 3)
    if H != Hkv:
        kh = np.repeat(kh, H // Hkv, axis=1)
        vh = np.repeat(vh, H // Hkv, axis=1)
    scores = np.matmul(qh, kh.transpose(0, 1, 3, 2)) / np.sqrt(Dh)
    mask = window_mask(S, layer.get("causal", False), layer.get("window_size"))
    if mask is not None:
        scores = scores + mask[None, None]
    m = np.max(scores, axis=-1, keepdims=True)
    e = np.exp(scores - m)
    attn = e / np.sum(e, axis=-1, keepdims=True)
    ctx = np.matmul(attn, vh).transpose(0, 2, 1, 3).reshape(B, S, E)
    return np.dot(ctx, layer["Wo"].T) + layer["bo"]


def router(x_flat: Any, layer: Dict[str, Any]) -> Tuple[Any, Any]:
    """Router logits and probabilities.  Follows ``nn/moe.py:23-28``."""
    logits = np.dot(x_flat, layer["Wr"].T) + layer["br"]
    e = np.exp(logits - np.max(logits, axis=-1, keepdims=True))
    return logits, e / np.sum(e, axis=-1, keepdims=True)


def top_k(probs: Any, k: int) -> Any:
    """Follows ``nn/moe.py:31-35``: a full argsort of ``-probs`` so ties
    resolve the same way every time."""
    return np.argsort(-probs, axis=-1)[:, :k]


forward_top_k = top_k


def moe_forward(x: Any, layer: Dict[str, Any],
                probs: Optional[Any] = None) -> Any:
    """Mixture-of-Experts forward.  Follows ``nn/moe.py:52-87`` minus the
    auxiliary loss (``:67-68``), which does not touch the output.

    ``probs`` overrides the router (the benchmark configuration draws router
    logits directly); ``None`` runs the layer's own router."""
    D = layer["embed_dim"]
    k = layer["top_k"]
    n_exp = layer["num_experts"]
    lead = x.shape[:-1]
    flat = x.reshape(-1, D)
    if probs is None:
        _, probs = router(flat, layer)
    chosen = top_k(probs, k)
    rows = np.arange(flat.shape[0])[:, None]
    gates = probs[rows, chosen]
    out = np.zeros_like(flat)
    for e in range(n_exp):
        tok, slot = np.nonzero(chosen == e)
        if tok.size == 0:
            continue
        xe = flat[tok]
        h = activate(layer["activation"], np.dot(xe, layer["W1"][e].T) + layer["b1"][e])
        y = np.dot(h, layer["W2"][e].T) + layer["b2"][e]
        np.add.at(out, tok, gates[tok, slot][:, None] * y)
    return out.reshape(lead + (D,))


def w8a8_dense(x: Any, w_codes: np.ndarray, w_scale: Any, bias: Any = None,
               activation: str = "linear") -> Tuple[Any, np.ndarray, Any, np.ndarray]:
    """Composed W8A8 Dense: ``(y, acc_int32, x_scale, x_codes)``.

    The reference has no integer GEMM (``compression/quantization.py:1-14``);
    this composes its own pieces: per-token symmetric 8-bit quantization of
    the activations is ``quantize_tensor(X, 8, "symmetric",
    per_channel=True)`` (``:76-93``, axis 0 = one scale per row), the codes
    are ``quantize`` (``:53-56``), the accumulator is the exact integer dot
    product of the codes, and ``y = acc * x_scale * w_scale.T + b`` followed
    by the activation (``nn/forward.py:318-321``).  ``acc`` is exact because
    |acc| <= 127 * 127 * K < 2^31 for K <= 133143, and it is formed in
    float64, which holds such integers exactly."""
    x = np.asarray(x, dtype=np.float32)
    _, x_scale, zp = quantize_tensor(x, 8, "symmetric", per_channel=True)
    x_codes = quantize(x, x_scale, zp, 8, "symmetric").astype(np.int8)
    acc = np.dot(x_codes.astype(np.float64), w_codes.astype(np.float64).T)
    acc = acc.astype(np.int32)
    ws = np.asarray(w_scale, dtype=np.float32).reshape(1, -1)
    y = (acc.astype(np.float32) * x_scale.astype(np.float32)) * ws
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return activate(activation, y), acc, x_scale, x_codes


def w8a8_static_dense(x: Any, spec: Dict[str, Any], w_codes: np.ndarray, w_scale: Any,
                      bias: Any = None, activation: str = "linear") -> Tuple[Any, np.ndarray, Any]:
    """Composed static W8A8 Dense: ``(y, acc_int32, x_codes)``.

    The activations take the calibrated per-tensor spec of the layer that
    produced them (``ActivationCalibrator``, ``compression/quantization.py:
    156-209``): ``q = quantize(x, scale, zero_point, bits, scheme)``
    (``:53-56``) in the dtype NumPy gives it; ``acc`` is the exact integer
    sum of ``(q - zero_point) * w_codes`` and ``y = act((acc * scale) *
    w_scale + b)`` in float32, evaluated in that order; for an ``x`` already
    fake-quantized by the spec, ``acc * scale * w_scale`` is the reference's
    ``x @ W.T`` (``nn/forward.py:318-319``) up to float rounding."""
    q = quantize(np.asarray(x, dtype=np.float32), spec["scale"], spec["zero_point"],
                 spec["bits"], spec["scheme"])
    zp = float(np.asarray(spec["zero_point"]).reshape(-1)[0])
    centred = q.astype(np.float64) - zp
    acc = np.dot(centred, w_codes.astype(np.float64).T).astype(np.int64)
    assert np.all(np.abs(acc) < 2 ** 31)
    acc = acc.astype(np.int32)
    ws = np.asarray(w_scale, dtype=np.float32).reshape(1, -1)
    s32 = np.float32(np.asarray(spec["scale"]).reshape(-1)[0])
    y = (acc.astype(np.float32) * s32) * ws
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)
    return activate(activation, y), acc, q


def forward(layers: List[Dict[str, Any]], inputs: Any,
            dtype: Any = np.float32) -> List[Any]:
    """Run the layer list; returns every layer's output (``outputs[0]`` is
    the input), as ``nn/forward.py:272-311,810-811`` does.  Covers the
    layer types of the benchmark configurations: dense, layernorm,
    multihead_attention (softmax, absolute positions), residual_save,
    residual_add, moe, and the decoding front end: embedding
    (``:414-422``), positional_encoding (``:597-603``), dropout at inference
    (``:398-413``); ``act_quant`` as ``forward.py:798-805``."""
    from .quantization import fake_quantize
    x = np.asarray(inputs, dtype=dtype)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    outputs = [x]
    for layer in layers:
        x = outputs[-1]
        kind = layer["type"]
        if kind in ("dense", "sparse"):
            x, _ = dense_forward(layer, x, dtype)
        elif kind == "layernorm":
            x = layernorm_forward(x, layer)
        elif kind == "multihead_attention":
            x = mha_forward(x, layer)
        elif kind == "residual_save":
            pass
        elif kind == "embedding":
            ids = np.asarray(x, dtype=np.int32)
            if ids.ndim == 1:
                ids = ids.reshape(-1, 1)
            x = layer["weights"][ids]
        elif kind == "positional_encoding":
            table = layer["weights"] if layer.get("_pos_type") == "learnable" else layer["pe"]
            x = x + table[:x.shape[1]][None, :, :]
        elif kind == "dropout":
            pass
        elif kind == "residual_add":
            x = x + outputs[layer["save_index"]]
        elif kind == "moe":
            x = moe_forward(x, layer)
        else:
            raise ValueError(f"Unknown layer type: {kind}")
        spec = layer.get("act_quant")
        if spec is not None:
            x = fake_quantize(x, spec["scale"], spec["zero_point"], spec["bits"], spec["scheme"])
        outputs.append(x)
    return outputs
