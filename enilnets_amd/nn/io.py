"""int8 on-disk format for quantized models.

The reference's ``Save`` writes the fake-quantized float weights
(``Enilnets/nn/io.py:61-112``), so a quantized model is as large on disk as
a float one.  ``SaveInt8`` writes each symmetric <= 8-bit float32 weight as
its int8 codes plus its ``quant`` spec, a quarter of the float32 bytes;
``LoadInt8`` restores the layer dicts exactly: the fake-quantized floats are
rebuilt on the device as ``code * scale`` (the same float32 product
``dequantize`` forms, ``compression/quantization.py:59-61``) and the codes go
straight into the layer's device int8 cache.

File: a NumPy ``.npz`` archive (read with ``allow_pickle=False``), entries
* ``meta``: UTF-8 JSON, ``{"format", "version", "layers": [...]}``; per layer
  its non-array values and the names of its arrays, int8 weights and specs;
* ``{i}/{key}``: float or other arrays, stored with their dtype;
* ``{i}/{key}/codes``: int8 codes in the weight's shape, -128 marking a code
  0 whose fake-quantized value is -0.0;
* ``{i}/quant/{key}/scale`` and ``/zero_point``, ``{i}/act_quant/scale``
  and ``/zero_point``: the spec values, with how to rebuild their type
  (0-d array, NumPy scalar or Python float) recorded in ``meta``.
Keys starting with ``_state_`` are transient and are skipped, as the
reference's ``Save`` skips them (``io.py:31-38``).
"""

import json
from typing import Any, Dict, Optional

import numpy as np

from .. import _lib
from ..device import DeviceArray
from .weights import Int8Weights, _row_scales, store_int8

FORMAT = "enilnets-amd-int8"
VERSION = 1
#: file code of an element whose code is 0 and whose fake-quantized value is
#: -0.0 (weight codes span [-127, 127], so -128 is free)
NEG_ZERO = -128


def _value_kind(v: Any) -> str:
    if isinstance(v, np.ndarray):
        return "array"
    if isinstance(v, np.generic):
        return "numpy"
    if isinstance(v, (float, int)) and not isinstance(v, bool):
        return "python"
    raise TypeError(f"spec value of type {type(v).__name__} is not supported")


def _restore_value(a: np.ndarray, kind: str) -> Any:
    if kind == "array":
        return a
    if kind == "numpy":
        return a[()]
    return a.item()


def _int8_eligible(value: np.ndarray, spec: Optional[Dict[str, Any]]) -> bool:
    return (spec is not None and spec.get("scheme") == "symmetric"
            and int(spec.get("bits", 32)) <= 8 and value.dtype == np.float32
            and value.ndim >= 2)


def _save_spec(arrays: Dict[str, np.ndarray], prefix: str, spec: Dict[str, Any]) -> Dict[str, Any]:
    out: Dict[str, Any] = {}
    for field, v in spec.items():
        if field in ("scale", "zero_point"):
            arrays[f"{prefix}/{field}"] = np.asarray(v)
            out[field] = {"kind": _value_kind(v)}
        else:
            out[field] = v
    return out


def _load_spec(z: Any, prefix: str, saved: Dict[str, Any]) -> Dict[str, Any]:
    spec: Dict[str, Any] = {}
    for field, v in saved.items():
        if field in ("scale", "zero_point"):
            spec[field] = _restore_value(z[f"{prefix}/{field}"], v["kind"])
        else:
            spec[field] = v
    return spec


def SaveInt8(model: Any, file: str) -> Dict[str, int]:
    """Write ``model.layers`` to ``file`` in the int8 format.  Returns
    ``{"int8_bytes", "float_bytes"}``: the bytes the int8 weights take and
    what the same weights take as floats."""
    from .weights import int8_weights
    meta: Dict[str, Any] = {"format": FORMAT, "version": VERSION, "layers": []}
    arrays: Dict[str, np.ndarray] = {}
    int8_bytes = float_bytes = 0
    for i, layer in enumerate(model.layers):
        specs = layer.get("quant", {})
        entry: Dict[str, Any] = {"order": [k for k in layer if not k.startswith("_state_")],
                                 "values": {}, "arrays": [], "int8": [], "quant": {}}
        for key, value in layer.items():
            if key.startswith("_state_") or key in ("quant", "act_quant"):
                continue
            if isinstance(value, np.ndarray):
                if _int8_eligible(value, specs.get(key)):
                    codes = int8_weights(layer, key).codes.numpy().reshape(value.shape)
                    # code 0 of a negative weight dequantizes to -0.0; the
                    # unused code -128 keeps that sign in the file
                    codes[(codes == 0) & np.signbit(value)] = NEG_ZERO
                    arrays[f"{i}/{key}/codes"] = codes
                    entry["int8"].append(key)
                    int8_bytes += codes.nbytes
                    float_bytes += value.nbytes
                else:
                    arrays[f"{i}/{key}"] = value
                    entry["arrays"].append(key)
            else:
                json.dumps(value)  # TypeError for values JSON cannot hold, as Save raises
                entry["values"][key] = value
        for name, spec in specs.items():
            entry["quant"][name] = _save_spec(arrays, f"{i}/quant/{name}", spec)
        if layer.get("act_quant") is not None:
            entry["act_quant"] = _save_spec(arrays, f"{i}/act_quant", layer["act_quant"])
        meta["layers"].append(entry)
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode("utf-8"), dtype=np.uint8)
    with open(file, "wb") as f:
        np.savez(f, **arrays)
    return {"int8_bytes": int8_bytes, "float_bytes": float_bytes}


def LoadInt8(file: str, model: Any = None) -> Any:
    """Read ``file`` into ``model.layers`` (a new ``Model`` when ``model`` is
    None) and return the model.  int8 weights come back as the
    fake-quantized floats plus their device int8 cache."""
    if model is None:
        from .model import Model
        model = Model()
    with np.load(file, allow_pickle=False) as z:
        meta = json.loads(bytes(z["meta"]).decode("utf-8"))
        if meta.get("format") != FORMAT or meta.get("version") != VERSION:
            raise ValueError(f"{file} is not a {FORMAT} v{VERSION} file")
        layers = []
        for i, entry in enumerate(meta["layers"]):
            layer: Dict[str, Any] = dict(entry["values"])
            for key in entry["arrays"]:
                layer[key] = z[f"{i}/{key}"]
            if entry["quant"]:
                layer["quant"] = {name: _load_spec(z, f"{i}/quant/{name}", saved)
                                  for name, saved in entry["quant"].items()}
            if "act_quant" in entry:
                layer["act_quant"] = _load_spec(z, f"{i}/act_quant", entry["act_quant"])
            for key in entry["int8"]:
                codes = np.array(z[f"{i}/{key}/codes"])
                neg_zero = codes == NEG_ZERO
                codes[neg_zero] = 0
                spec = layer["quant"][key]
                rows = _row_scales(codes.shape, spec["scale"])
                d_codes, d_rows = DeviceArray.from_numpy(codes), DeviceArray.from_numpy(rows)
                fake = DeviceArray(codes.shape, np.float32)
                _lib.call("enq_dequantize_i8", _lib.F32, d_codes.ptr, 1, rows.size,
                          codes.size // rows.size, d_rows.ptr, fake.ptr)
                host = fake.numpy()
                host[neg_zero] = -0.0
                layer[key] = host
                store_int8(layer, key, Int8Weights(d_codes, d_rows, codes.shape,
                                                   int(spec["bits"]), np.size(spec["scale"]) > 1,
                                                   layer[key], spec["scale"]))
            layers.append({k: layer[k] for k in entry["order"]})
    model.layers = layers
    return model


__all__ = ["SaveInt8", "LoadInt8", "FORMAT", "VERSION"]
