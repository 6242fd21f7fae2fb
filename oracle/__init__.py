"""CPU oracle for the quantized-inference hot path.

TEST INFRASTRUCTURE ONLY.  This package restates, in plain NumPy, the
reference algorithm (Enilnets v4.11.0, ``Enilnets/compression/quantization.py``
and the Dense / MoE / attention-projection branches of ``Enilnets/nn``) so the
HIP implementation in ``enilnets_amd`` can be checked against it.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU
baseline.  The product path (``enilnets_amd``) never imports, calls or falls
back to anything in here.

Pinning status of each function (what checks it besides being a restatement)
is listed in ``oracle/PINNING.md``.
"""

from .quantization import (QUANTIZABLE, compute_scale, dequantize,
                           fake_quantize, quant_range, quantization_error,
                           quantize, quantize_tensor, quantize_weights,
                           int8_codes)
from .qat import MovingRange, qat_linear_forward, qat_quantized_weight, ste_mask
from .calibration import observe_ranges, percentile, specs_from_ranges
from .forward import (activate, dense_forward, forward, forward_top_k, layernorm_forward,
                      mha_forward, moe_forward, router, top_k, w8a8_dense, w8a8_static_dense,
                      window_mask)

__all__ = [
    "QUANTIZABLE", "compute_scale", "dequantize", "fake_quantize",
    "quant_range", "quantization_error", "quantize", "quantize_tensor",
    "quantize_weights", "int8_codes", "activate", "dense_forward", "forward",
    "layernorm_forward", "mha_forward", "moe_forward", "w8a8_dense", "w8a8_static_dense", "forward_top_k",
    "router", "top_k", "window_mask", "MovingRange", "qat_linear_forward",
    "qat_quantized_weight", "ste_mask", "observe_ranges", "percentile", "specs_from_ranges",
]
