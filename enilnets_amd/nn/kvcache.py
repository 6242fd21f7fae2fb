"""KV-cache incremental decoding on the device (``Enilnets/nn/kvcache.py``).

``cached_forward_step`` steps new tokens (token ids through an embedding
layer, or float activations) through a causal stack and returns the outputs
at the new positions only, as ``kvcache.py:66-118`` does.  Every projection
runs as a W8 Dense with M = batch x new tokens, which for decoding is the
split-K GEMV; attention runs ``enq_attention_kv`` over the cached keys and
values plus the new ones.

The cache keeps, per attention layer, K and V of the un-expanded K/V heads
in device buffers laid out ``(batch, capacity, kv_heads * head_dim)``, the
absolute position of the oldest kept entry, and the count of live entries.
A sliding window evicts entries no query of the step can see again
(``kvcache.py:158-175``); the buffer is compacted into a new one when an
append would run past its capacity, so memory stays bounded by the window.

Layer types: embedding, positional_encoding, layernorm, dense, dropout
(inference no-op), residual_save / residual_add, moe and causal softmax
multi-head attention with absolute positions (MHA, MQA, GQA, window).
"""

from typing import Any, Dict, Optional

import numpy as np

from .. import _lib
from ..device import DeviceArray, null
from .dense import dense_w8
from .forward import _FLOAT64_ACTIVATIONS, _bias
from .moe import moe_forward
from .transformer import (MhaPlan, _at, _check_supported, embedding, layernorm, layernorm_params,
                          positional_encoding)
from .weights import int8_weights


class _KV:
    """Cached keys and values of one attention layer."""

    def __init__(self, batch: int, width: int, capacity: int):
        self.batch, self.width, self.capacity = batch, width, capacity
        self.k = DeviceArray((batch, capacity, width), np.float32)
        self.v = DeviceArray((batch, capacity, width), np.float32)
        self.base = 0      # buffer row of the oldest live entry
        self.length = 0    # live entries
        self.start = 0     # absolute position of the oldest live entry

    def reserve(self, extra: int) -> None:
        """Room for ``extra`` more rows after the live ones, compacting or
        growing into a fresh buffer when needed."""
        if self.base + self.length + extra <= self.capacity:
            return
        cap = max(64, 2 * (self.length + extra))
        k = DeviceArray((self.batch, cap, self.width), np.float32)
        v = DeviceArray((self.batch, cap, self.width), np.float32)
        for src, dst in ((self.k, k), (self.v, v)):
            _lib.call("enq_copy_rows", _at(src, 4 * self.base * self.width), self.width,
                      self.capacity, null(), dst.ptr, self.width, cap, self.length,
                      self.width, self.batch)
        self.k, self.v, self.capacity, self.base = k, v, cap, 0

    def gather_batch(self, index: np.ndarray) -> None:
        """New batch row b takes old row index[b] (beam search)."""
        idx = DeviceArray.from_numpy(np.ascontiguousarray(index, dtype=np.int32))
        n = int(index.size)
        row = self.capacity * self.width
        k = DeviceArray((n, self.capacity, self.width), np.float32)
        v = DeviceArray((n, self.capacity, self.width), np.float32)
        for src, dst in ((self.k, k), (self.v, v)):
            _lib.call("enq_copy_rows", src.ptr, row, 0, idx.ptr, dst.ptr, row, 0, n, row, 1)
        self.k, self.v, self.batch = k, v, n


class KVCache:
    """Per-stream decoding state (``kvcache.py:23-64``): cached K/V per
    attention layer, cached residual-save activations, and the absolute
    position of the next token.

    ``trust_weights`` (not in the reference) is a promise that the model's
    weight and bias arrays are not modified in place during the session:
    each step then reuses the layers' device weights, biases, LayerNorm
    parameters and attention buffers instead of re-validating the int8
    weights against the host arrays (a full hash of every weight per step)
    and uploading the biases and LayerNorm parameters again.  Arrays
    replaced by new objects are still picked up."""

    def __init__(self, trust_weights: bool = False) -> None:
        self.kv: Dict[int, _KV] = {}
        self.residual: Dict[int, DeviceArray] = {}
        self.residual_dtype: Dict[int, Any] = {}  # host dtype the reference would hold
        self.position: int = 0
        self.trust_weights = bool(trust_weights)
        self._resources: Dict[Any, Any] = {}  # trusted sessions: per-layer device resources

    def __repr__(self) -> str:
        return f"KVCache(position={self.position}, attention_layers={sorted(self.kv)})"

    def reorder(self, index: Any) -> None:
        """Gather every cached tensor along the batch axis by ``index``."""
        idx = np.asarray(index, dtype=np.int64).reshape(-1)
        for entry in self.kv.values():
            if np.any((idx < 0) | (idx >= entry.batch)):
                raise IndexError(f"batch index out of range for a cache of {entry.batch} rows")
            entry.gather_batch(idx)
        for key, value in list(self.residual.items()):
            if np.any((idx < 0) | (idx >= value.shape[0])):
                raise IndexError(f"batch index out of range for {value.shape[0]} rows")
            width = value.size // value.shape[0]
            d_idx = DeviceArray.from_numpy(idx.astype(np.int32))
            out = DeviceArray((idx.size,) + value.shape[1:], np.float32)
            _lib.call("enq_copy_rows", value.ptr, width, 0, d_idx.ptr, out.ptr, width, 0,
                      idx.size, width, 1)
            self.residual[key] = out

    def expand(self, size: int) -> None:
        """Replicate a batch-1 cache to ``size`` rows."""
        self.reorder([0] * int(size))


def _layer_ids(layer: Dict[str, Any]) -> tuple:
    return tuple(id(v) for v in layer.values() if isinstance(v, np.ndarray))


def _resources(cache: KVCache, key: Any, layer: Dict[str, Any], make: Any) -> Any:
    """``make()``, or in a trusted session the result kept for ``key`` while
    the layer's arrays are the same objects."""
    if not cache.trust_weights:
        return make()
    ids = _layer_ids(layer)
    kept = cache._resources.get(key)
    if kept is None or kept[0] != ids:
        kept = (ids, make())
        cache._resources[key] = kept
    return kept[1]


def _attention_step(x: DeviceArray, layer: Dict[str, Any], idx: int, cache: KVCache,
                    pos: int, variant: str) -> DeviceArray:
    """kvcache.py:121-213 for the softmax, absolute-position branch."""
    if not layer.get("causal", False):
        raise ValueError(
            f"KV-cache stepping requires causal attention; layer {idx} is non-causal (its full "
            "output at earlier positions would change when later tokens arrive, which a cache "
            "cannot represent).")
    _check_supported(layer, False)
    B, S_new, _ = x.shape
    plan = _resources(cache, ("mha", idx, B, S_new), layer, lambda: MhaPlan(layer, B, S_new))
    n_all = plan.wqkv.shape[0]
    dense_w8(x, plan.wqkv, plan.bqkv, "linear", variant=variant, out=plan.qkv)
    entry = cache.kv.get(idx)
    if entry is None or entry.batch != B:
        if entry is not None:
            raise ValueError(f"cache holds batch {entry.batch}, step has batch {B}")
        entry = _KV(B, plan.nkv, max(64, 2 * S_new))
        entry.start = pos
        cache.kv[idx] = entry
    entry.reserve(S_new)
    row0 = entry.base + entry.length
    for dst, col in ((entry.k, plan.nq), (entry.v, plan.nq + plan.nkv)):
        _lib.call("enq_copy_rows", _at(plan.qkv, 4 * col), n_all, S_new, null(),
                  _at(dst, 4 * row0 * plan.nkv), plan.nkv, entry.capacity, S_new, plan.nkv, B)
    entry.length += S_new
    if plan.window >= 0:
        # keep what the oldest query of this step can still see
        drop = max(0, (pos - plan.window) - entry.start)
        drop = min(drop, entry.length - S_new)
        entry.base += drop
        entry.length -= drop
        entry.start += drop
    _lib.call("enq_attention_kv", plan.qkv.ptr, n_all, S_new, S_new, pos,
              _at(entry.k, 4 * entry.base * plan.nkv), plan.nkv,
              _at(entry.v, 4 * entry.base * plan.nkv), plan.nkv, entry.capacity, entry.length,
              entry.start, B, plan.H, plan.Hkv, plan.Dh, 1, plan.window, plan.ctx.ptr, plan.nq)
    return dense_w8(plan.ctx, plan.wo, plan.bo, "linear", variant=variant)


def cached_forward_step(model: Any, inputs: Any, cache: KVCache, advance_position: bool = True,
                        variant: str = "fp32") -> np.ndarray:
    """Step ``inputs`` -- token ids ``(batch, n_new)`` (or ``(n_new,)`` as
    batch 1) for a model starting with an embedding layer, else float
    activations ``(batch, n_new, width)`` -- through ``model.layers``,
    reading and updating ``cache``.  Returns ``(batch, n_new, out_dim)`` for
    the new positions (``kvcache.py:66-118``)."""
    layers = model.layers
    pos = cache.position
    if layers and layers[0]["type"] == "embedding":
        ids = np.asarray(inputs)
        if ids.ndim == 1:
            ids = ids[None, :]
        x = None
    else:
        host = np.asarray(inputs, dtype=np.float32)
        if host.ndim == 2:
            host = host[None]
        x = DeviceArray.from_numpy(host)
    dtype: Any = np.float32
    for idx, layer in enumerate(layers):
        t = layer["type"]
        if t == "embedding":
            if x is not None:
                raise NotImplementedError("an embedding layer after the first is not supported")
            x = embedding(ids, layer)
            dtype = np.asarray(layer["weights"]).dtype
        elif t == "positional_encoding":
            x = positional_encoding(x, layer, pos)
        elif t == "layernorm":
            # gamma and beta uploaded once per trusted session (each upload
            # is a synchronous copy that waits for the queued kernels)
            params = _resources(cache, ("layernorm", idx), layer,
                                lambda layer=layer: layernorm_params(layer))
            x = layernorm(x, layer, params=params)
            dtype = np.result_type(dtype, np.asarray(layer["gamma"]).dtype,
                                   np.asarray(layer["beta"]).dtype)
        elif t == "dense":
            def make(layer=layer):
                w = int8_weights(layer, "weights")
                return w, _bias(layer, "bias", w.shape[0])
            w, b = _resources(cache, ("dense", idx), layer, make)
            dtype = np.float64 if layer["activation"] in _FLOAT64_ACTIVATIONS else np.float32
            # no act_quant: the reference's cached step never fake-quantizes
            # layer outputs (kvcache.py:84-118), calibrated or not
            x = dense_w8(x, w, b, layer["activation"],
                         layer.get("activation_params", {}), variant, out_dtype=dtype)
        elif t == "dropout":
            pass
        elif t == "residual_save":
            cache.residual[idx] = x
            cache.residual_dtype[idx] = dtype
        elif t == "residual_add":
            saved = cache.residual[layer["save_index"]]
            y = DeviceArray(x.shape, np.float32)
            _lib.call("enq_add", x.ptr, saved.ptr, x.size, y.ptr)
            x = y
            dtype = np.result_type(dtype, cache.residual_dtype[layer["save_index"]])
        elif t == "moe":
            x, _ = moe_forward(x, layer, variant, aux_loss=False)
        elif t == "multihead_attention":
            x = _attention_step(x, layer, idx, cache, pos, variant)
            dtype = np.float64
        else:
            raise ValueError(
                f"KV-cache stepping doesn't support layer type '{t}' (layer {idx}); use a full "
                "Forward() for this architecture.")
    if advance_position:
        cache.position += int(x.shape[1])
    out = x.numpy()
    return out if out.dtype == dtype else out.astype(dtype)
