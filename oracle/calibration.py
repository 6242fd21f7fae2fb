"""NumPy restatement of ``ActivationCalibrator`` (activation ranges).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): never imported by the
product package.

Follows ``Enilnets/compression/quantization.py:156-209``: ``observe`` widens
each floating layer output's recorded range, either the global min / max or,
with a percentile p, ``np.percentile(out, 100 - p)`` and ``np.percentile(out,
p)`` (NumPy's default 'linear' method, ``:183-188``); ``apply`` turns every
range into a spec through ``compute_scale``.
"""

from typing import Any, Dict, List, Optional, Sequence

import numpy as np

from .quantization import compute_scale


def percentile(out: Any, q: float) -> float:
    """``float(np.percentile(out, q))``, the reference's own expression."""
    return float(np.percentile(out, q))


def observe_ranges(outputs: Sequence[Any], percentile_p: Optional[float] = None,
                   ranges: Optional[Dict[int, List[float]]] = None) -> Dict[int, List[float]]:
    """One ``observe`` step over ``outputs`` (``outputs[i + 1]`` is layer i's
    output, as ``Forward`` leaves them); ``quantization.py:176-192``."""
    ranges = {} if ranges is None else ranges
    for i in range(len(outputs) - 1):
        out = outputs[i + 1]
        if not hasattr(out, "dtype") or out.dtype.kind != "f":
            continue
        if percentile_p is None:
            low, high = float(np.min(out)), float(np.max(out))
        else:
            low = percentile(out, 100.0 - percentile_p)
            high = percentile(out, percentile_p)
        if i in ranges:
            ranges[i] = [min(ranges[i][0], low), max(ranges[i][1], high)]
        else:
            ranges[i] = [low, high]
    return ranges


def specs_from_ranges(ranges: Dict[int, List[float]], bits: int = 8,
                      scheme: str = "asymmetric") -> Dict[int, Dict[str, Any]]:
    """``apply`` without the model: ``quantization.py:194-209``."""
    if not ranges:
        raise RuntimeError("no calibration data observed -- call observe(X) first")
    specs = {}
    for i, (low, high) in ranges.items():
        scale, zero_point = compute_scale(np.asarray(low), np.asarray(high), bits, scheme)
        specs[i] = {"bits": bits, "scheme": scheme, "scale": scale, "zero_point": zero_point,
                    "low": low, "high": high}
    return specs
