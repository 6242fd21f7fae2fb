"""Device-resident transformer-block layers of the quantized path.

* ``layernorm`` follows ``Enilnets/nn/forward.py:207-254`` (2-D and 3-D
  inputs: statistics over the last axis);
* ``residual_add`` follows ``forward.py:762-766``;
* ``mha_forward`` follows the softmax branch of the multi-head attention
  layer, ``forward.py:423-436,525-551``: the Q, K and V projections run as one
  W8 Dense over the row-concatenated int8 codes of ``Wq``, ``Wk`` and ``Wv``,
  the attention core as one HIP kernel reading the fused projection output
  in place, and the output projection as a W8 Dense on ``Wo``.
"""

import ctypes
from typing import Any, Dict, Optional, Tuple

import numpy as np

from .. import _lib
from ..device import DeviceArray
from .dense import dense_w8
from .weights import _CACHE_KEY, Int8Weights, int8_weights

#: Entry of the layer's int8 cache holding the fused projection; it keeps
#: the three weights it was built from, so a rebuilt one is noticed.
_QKV_KEY = "_qkv"


def _at(a: DeviceArray, byte_offset: int) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.address + byte_offset)


def layernorm(x: DeviceArray, layer: Dict[str, Any], out: Optional[DeviceArray] = None,
              params: Optional[Tuple[DeviceArray, DeviceArray]] = None) -> DeviceArray:
    """LayerNorm of a ``(..., E)`` float32 device array over its last axis
    with the layer's ``gamma``, ``beta`` and ``epsilon``.  ``params`` passes
    gamma and beta already on the device."""
    if len(x.shape) not in (2, 3):
        raise NotImplementedError(
            f"LayerNorm on the quantized path takes 2-D or 3-D inputs, got {len(x.shape)}-D")
    e = x.shape[-1]
    if params is None:
        params = layernorm_params(layer)
    d_g, d_b = params
    if d_g.size != e or d_b.size != e:
        raise ValueError(f"gamma/beta of size {d_g.size}/{d_b.size} do not match width {e}")
    y = out if out is not None else DeviceArray(x.shape, np.float32)
    _lib.call("enq_layernorm", x.ptr, x.size // e, e, d_g.ptr, d_b.ptr,
              float(layer.get("epsilon", 1e-5)), y.ptr)
    return y


def layernorm_params(layer: Dict[str, Any]) -> Tuple[DeviceArray, DeviceArray]:
    """The layer's gamma and beta as float32 device vectors."""
    gamma = np.ascontiguousarray(layer["gamma"], dtype=np.float32).reshape(-1)
    beta = np.ascontiguousarray(layer["beta"], dtype=np.float32).reshape(-1)
    return DeviceArray.from_numpy(gamma), DeviceArray.from_numpy(beta)


def residual_add(x: DeviceArray, saved: DeviceArray,
                 out: Optional[DeviceArray] = None) -> DeviceArray:
    """``x + saved`` for float32 device arrays of one shape."""
    if tuple(x.shape) != tuple(saved.shape):
        raise ValueError(f"operands could not be broadcast together with shapes "
                         f"{x.shape} {saved.shape}")
    y = out if out is not None else DeviceArray(x.shape, np.float32)
    _lib.call("enq_add", x.ptr, saved.ptr, x.size, y.ptr)
    return y


def token_rows(tokens: Any, vocab: int) -> np.ndarray:
    """Token ids as the embedding rows NumPy indexing would read
    (``forward.py:414-422``): int32 ids, negative ids counted from the end,
    IndexError outside ``[-vocab, vocab)``; a 1-D input is one token per row."""
    ids = np.asarray(tokens, dtype=np.int32)
    if ids.ndim == 1:
        ids = ids.reshape(-1, 1)
    bad = (ids < -vocab) | (ids >= vocab)
    if bad.any():
        raise IndexError(f"index {int(ids[bad].reshape(-1)[0])} is out of bounds for axis 0 "
                         f"with size {vocab}")
    return np.ascontiguousarray(np.where(ids < 0, ids + vocab, ids), dtype=np.int32)


def embedding(tokens: Any, layer: Dict[str, Any]) -> DeviceArray:
    """``layer["weights"][ids]`` gathered on the device."""
    from .weights import device_table
    table = device_table(layer, "weights")
    vocab, width = table.shape
    ids = token_rows(tokens, vocab)
    d_ids = DeviceArray.from_numpy(ids)
    out = DeviceArray(ids.shape + (width,), np.float32)
    _lib.call("enq_copy_rows", table.ptr, width, 0, d_ids.ptr, out.ptr, width, 0, ids.size,
              width, 1)
    return out


def positional_encoding(x: DeviceArray, layer: Dict[str, Any], pos: int = 0,
                        out: Optional[DeviceArray] = None) -> DeviceArray:
    """``x + table[pos:pos+S][None]`` (``forward.py:597-603``; a KV-cache
    step passes its first absolute position, ``kvcache.py:88-91``)."""
    from .weights import device_table
    if len(x.shape) != 3:
        raise ValueError(f"positional encoding expects (batch, seq, embed), got {x.shape}")
    key = "weights" if layer.get("_pos_type") == "learnable" else "pe"
    table = device_table(layer, key)
    B, S, E = x.shape
    if table.shape[1] != E:
        raise ValueError(f"table width {table.shape[1]} does not match {E}")
    if pos + S > table.shape[0]:
        raise ValueError(f"operands could not be broadcast together: positions {pos}..{pos + S} "
                         f"of a {table.shape[0]}-row table")
    y = out if out is not None else DeviceArray(x.shape, np.float32)
    _lib.call("enq_add_bcast", x.ptr, _at(table, 4 * pos * E), B, S * E, y.ptr)
    return y


def _fused_qkv(layer: Dict[str, Any]) -> Tuple[Int8Weights, int, int]:
    """int8 codes and row scales of ``[Wq; Wk; Wv]`` in one device buffer,
    rebuilt whenever one of the three cached weights is."""
    parts = tuple(int8_weights(layer, name) for name in ("Wq", "Wk", "Wv"))
    cache = layer[_CACHE_KEY]  # int8_weights created it
    cached = cache.get(_QKV_KEY)
    if (cached is not None and cached[1] is not None
            and all(a is b for a, b in zip(cached[0], parts))):
        return cached[1], parts[0].shape[0], parts[1].shape[0]
    k = parts[0].shape[1]
    if any(len(p.shape) != 2 or p.shape[1] != k for p in parts):
        raise ValueError("Wq, Wk and Wv must be 2-D with the same input width")
    rows = sum(p.shape[0] for p in parts)
    codes = DeviceArray((rows, k), np.int8)
    scale = DeviceArray((rows,), np.float32)
    r = 0
    for p in parts:
        n = p.shape[0]
        _lib.call("enq_copy_on_device", _at(codes, r * k), p.codes.ptr, n * k)
        _lib.call("enq_copy_on_device", _at(scale, 4 * r), p.scale.ptr, 4 * n)
        r += n
    fused = Int8Weights(codes, scale, (rows, k), parts[0].bits, True, None, None)
    cache[_QKV_KEY] = (parts, fused)
    return fused, parts[0].shape[0], parts[1].shape[0]


def _vector(layer: Dict[str, Any], key: str, n: int) -> np.ndarray:
    b = layer.get(key)
    if b is None:
        return np.zeros(n, np.float32)
    return np.ascontiguousarray(b, dtype=np.float32).reshape(-1)


def _check_supported(layer: Dict[str, Any], training: bool) -> None:
    if layer.get("attention_kernel", "softmax") != "softmax":
        raise NotImplementedError("only the softmax attention kernel is on the quantized path")
    if layer.get("positional_scheme", "absolute") != "absolute":
        raise NotImplementedError("rope/alibi positions are not on the quantized path")
    if layer.get("sparse_pattern") is not None:
        raise NotImplementedError("block-sparse attention is not on the quantized path")
    if training and layer.get("dropout", 0.0) > 0:
        raise NotImplementedError("attention dropout (training) is not on the quantized path")


class MhaPlan:
    """Device resources of one attention layer at one input shape: the fused
    QKV weights and biases, the output projection and the intermediate
    buffers.  Reusing a plan across calls keeps them allocated."""

    def __init__(self, layer: Dict[str, Any], batch: int, seq: int):
        self.H = int(layer["num_heads"])
        self.Dh = int(layer["head_dim"])
        hkv = layer.get("num_kv_heads")
        self.Hkv = self.H if hkv is None else int(hkv)
        self.wqkv, self.nq, self.nkv = _fused_qkv(layer)
        if self.nq != self.H * self.Dh or self.nkv != self.Hkv * self.Dh:
            raise ValueError(f"projection widths {self.nq}/{self.nkv} do not match heads "
                             f"{self.H}x{self.Dh}/{self.Hkv}x{self.Dh}")
        self.wo = int8_weights(layer, "Wo")
        bias = np.concatenate([_vector(layer, "bq", self.nq), _vector(layer, "bk", self.nkv),
                               _vector(layer, "bv", self.nkv)])
        self.bqkv = DeviceArray.from_numpy(bias)
        self.bo = DeviceArray.from_numpy(_vector(layer, "bo", self.wo.shape[0]))
        self.batch, self.seq = batch, seq
        self.qkv = DeviceArray((batch, seq, self.wqkv.shape[0]), np.float32)
        self.ctx = DeviceArray((batch, seq, self.nq), np.float32)
        self.causal = 1 if layer.get("causal", False) else 0
        window = layer.get("window_size")
        self.window = -1 if window is None else int(window)


def mha_forward(x: DeviceArray, layer: Dict[str, Any], variant: str = "fp32",
                training: bool = False, plan: Optional[MhaPlan] = None,
                out: Optional[DeviceArray] = None) -> DeviceArray:
    """Multi-head self-attention of a ``(B, S, E)`` float32 device array on
    the layer's int8 projection weights.  ``tiled_block_size`` computes the
    same numbers as the plain softmax (``forward.py:496-500``) and takes the
    same kernel."""
    _check_supported(layer, training)
    if len(x.shape) != 3:
        raise ValueError(f"multihead_attention expects (batch, seq, embed) input, got {x.shape}")
    B, S, _ = x.shape
    if plan is None:
        plan = MhaPlan(layer, B, S)
    elif (plan.batch, plan.seq) != (B, S):
        raise ValueError(f"plan made for ({plan.batch}, {plan.seq}), input is ({B}, {S})")
    n_all = plan.wqkv.shape[0]
    dense_w8(x, plan.wqkv, plan.bqkv, "linear", variant=variant, out=plan.qkv)
    _lib.call("enq_attention", plan.qkv.ptr, n_all, _at(plan.qkv, 4 * plan.nq), n_all,
              _at(plan.qkv, 4 * (plan.nq + plan.nkv)), n_all, B, S, plan.H, plan.Hkv, plan.Dh,
              plan.causal, plan.window, plan.ctx.ptr, plan.nq)
    return dense_w8(plan.ctx, plan.wo, plan.bo, "linear", variant=variant, out=out)
