"""Drop-in for ``Enilnets.compression``'s quantization exports
(``Enilnets/compression/__init__.py:9-12``), running on MI355X."""

from .quantization import (QUANTIZABLE, ActivationCalibrator, compute_scale, dequantize,
                           fake_quantize, quant_range, quantization_error, quantize,
                           quantize_tensor, quantize_weights, remove_activation_quantization)

__all__ = [
    "quantize_weights", "ActivationCalibrator", "quantize_tensor", "fake_quantize",
    "quantize", "dequantize", "compute_scale", "quant_range", "quantization_error",
    "remove_activation_quantization", "QUANTIZABLE",
]
