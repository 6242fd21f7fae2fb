"""Device-resident int8 weights of a quantized layer.

The reference keeps quantized weights as fake-quantized floats in the layer
dict (``Enilnets/compression/quantization.py:138-141``).  The integer kernels
need the int8 codes and per-channel scales in HBM; this module keeps them in
``layer["_state_enq_int8"][name]``.  ``_state_`` keys are excluded from
``Save`` (``Enilnets/nn/io.py:31-38``), and a deep copy of the layer
(``NeuralNet.copy``, ``core/base.py:233``) drops the cache instead of sharing
device memory.

A cache entry remembers which host array it was made from (object identity
plus a content hash of the array and its scale), so an array that was
replaced or modified in place is detected and its codes are rebuilt from the
fake-quantized floats with the stored scale (``enq_quantize`` semantics,
exact because |code| <= 127 keeps ``w_fq / scale`` within 1e-5 of the code).
"""

import ctypes
from typing import Any, Dict, Optional

import numpy as np

from .. import _lib
from ..device import DeviceArray

_CACHE_KEY = "_state_enq_int8"

try:
    import xxhash as _xxhash

    def _digest(a: np.ndarray) -> int:
        return _xxhash.xxh3_64_intdigest(np.ascontiguousarray(a).view(np.uint8))
except ImportError:  # pragma: no cover - image always has xxhash
    import zlib

    def _digest(a: np.ndarray) -> int:
        return zlib.crc32(np.ascontiguousarray(a).view(np.uint8))


class Int8Weights:
    """int8 codes ``(rows, cols)`` (or stacked ``(E, rows, cols)``) plus one
    fp32 scale per output row, resident on the device."""

    __slots__ = ("codes", "scale", "shape", "bits", "per_channel", "source_id",
                 "source_digest", "_code_sums")

    def __init__(self, codes: DeviceArray, scale: DeviceArray, shape, bits: int,
                 per_channel: bool, source: Optional[np.ndarray], scale_host: Any):
        self.codes = codes
        self.scale = scale
        self.shape = tuple(shape)
        self.bits = bits
        self.per_channel = per_channel
        self.source_id = id(source) if source is not None else None
        self.source_digest = (_digest(source) ^ _digest(np.asarray(scale_host, np.float32))
                              if source is not None else None)
        self._code_sums = None

    @property
    def code_sums(self) -> DeviceArray:
        """Per output row, the sum of its int8 codes (int32, device), made
        once: the zero-point term of static W8A8."""
        if self._code_sums is None:
            rows, k = self.shape[-2], self.shape[-1]
            sums = DeviceArray((rows,), np.int32)
            _lib.call("enq_code_row_sums", self.codes.ptr, rows, k, sums.ptr)
            self._code_sums = sums
        return self._code_sums

    def __deepcopy__(self, memo):
        return None

    def matches(self, source: np.ndarray, scale_host: Any) -> bool:
        if self.source_id != id(source):
            return False
        return self.source_digest == (_digest(source) ^ _digest(np.asarray(scale_host,
                                                                            np.float32)))

    @classmethod
    def from_device(cls, fake: np.ndarray, scale_host: np.ndarray, d_codes: DeviceArray,
                    d_scale: DeviceArray, per_channel: bool, bits: int) -> "Int8Weights":
        """Wrap codes produced by ``enq_quantize_tensor``; the scale is
        expanded to one value per output row."""
        shape = fake.shape
        rows = _row_scales(shape, scale_host)
        d_rows = d_scale if d_scale.size == rows.size else DeviceArray.from_numpy(rows)
        return cls(d_codes, d_rows, shape, bits, per_channel, fake, scale_host)

    @classmethod
    def from_fake(cls, fake: np.ndarray, spec: Dict[str, Any]) -> "Int8Weights":
        """Rebuild codes from fake-quantized floats and their stored scale."""
        if spec.get("scheme") != "symmetric" or int(spec.get("bits", 8)) > 8:
            raise NotImplementedError(
                "the integer Dense kernels take symmetric weights of at most 8 bits; got "
                f"scheme={spec.get('scheme')!r} bits={spec.get('bits')}")
        fake = np.asarray(fake)
        if fake.dtype != np.float32:
            raise NotImplementedError(
                f"the W8 Dense kernels take float32 layers, got {fake.dtype}")
        scale_host = np.asarray(spec["scale"])
        rows = _row_scales(fake.shape, scale_host)
        bits = int(spec["bits"])
        qmax = 2 ** (bits - 1) - 1
        n_rows = rows.size
        d_fake = DeviceArray.from_numpy(fake)
        d_rows = DeviceArray.from_numpy(rows)
        d_zero = DeviceArray.from_numpy(np.zeros(n_rows, np.float32))
        d_codes = DeviceArray(fake.shape, np.int8)
        _lib.call("enq_quantize_codes_i8", _lib.F32, d_fake.ptr, 1, n_rows,
                  fake.size // n_rows, d_rows.ptr, d_zero.ptr, -qmax, qmax, d_codes.ptr)
        return cls(d_codes, d_rows, fake.shape, bits, scale_host.size > 1, fake, scale_host)


def _row_scales(shape, scale_host) -> np.ndarray:
    """One fp32 scale per output row of a (rows, cols) or (E, rows, cols)
    weight, from a per-tensor, per-row or per-expert scale array."""
    scale = np.asarray(scale_host, dtype=np.float32)
    lead = shape[:-1]
    n_rows = int(np.prod(lead, dtype=np.int64))
    if scale.size == 1:
        return np.full(n_rows, scale.reshape(-1)[0], np.float32)
    padded = scale.reshape(scale.shape + (1,) * (len(shape) - scale.ndim))
    return np.ascontiguousarray(np.broadcast_to(padded[..., 0], lead).reshape(-1),
                                dtype=np.float32)


def store_int8(layer: Dict[str, Any], name: str, weights: Int8Weights) -> None:
    cache = layer.get(_CACHE_KEY)
    if cache is None:
        cache = {}
        layer[_CACHE_KEY] = cache
    cache[name] = weights


def int8_weights(layer: Dict[str, Any], name: str) -> Int8Weights:
    """The device codes of ``layer[name]``, rebuilt if the cache is missing
    or stale.  Raises NotImplementedError for a layer that was never
    quantized: the integer kernels have no float-weight path."""
    spec = layer.get("quant", {}).get(name)
    if spec is None:
        raise NotImplementedError(
            f"layer weight {name!r} is not quantized; run quantize_weights(model) first "
            "(enilnets_amd runs Dense layers on int8 weights only)")
    source = layer[name]
    cache = layer.get(_CACHE_KEY) or {}
    entry = cache.get(name)
    if entry is not None and entry.matches(source, spec["scale"]):
        return entry
    entry = Int8Weights.from_fake(source, spec)
    store_int8(layer, name, entry)
    return entry


_TABLE_KEY = "_state_enq_tables"


class DeviceTable:
    """A float32 device copy of a layer's float table (embedding and
    positional tables), checked against its host array like the int8 cache."""

    __slots__ = ("data", "source_id", "source_digest")

    def __init__(self, host: np.ndarray):
        self.data = DeviceArray.from_numpy(np.ascontiguousarray(host, dtype=np.float32))
        self.source_id = id(host)
        self.source_digest = _digest(host)

    def __deepcopy__(self, memo):
        return None

    def matches(self, host: np.ndarray) -> bool:
        return self.source_id == id(host) and self.source_digest == _digest(host)


def device_table(layer: Dict[str, Any], name: str) -> DeviceArray:
    """``layer[name]`` as a float32 device array, uploaded again only when
    the host array was replaced or changed."""
    host = np.asarray(layer[name])
    if host.dtype != np.float32:
        raise NotImplementedError(f"{name} of dtype {host.dtype}: the device path takes "
                                  "float32 tables")
    cache = layer.get(_TABLE_KEY)
    if cache is None:
        cache = {}
        layer[_TABLE_KEY] = cache
    entry = cache.get(name)
    if entry is None or not entry.matches(layer[name]):
        entry = DeviceTable(layer[name])
        cache[name] = entry
    return entry.data
