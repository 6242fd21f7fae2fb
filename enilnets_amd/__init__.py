"""enilnets_amd: Enilnets' quantized-inference hot path on AMD MI355X.

A drop-in for ``Enilnets.compression``'s quantization functions and for the
Dense ``Forward`` of quantized models, computed by hand-written gfx950 HIP
kernels in ``libenilnets_amd.so`` (C ABI: ``include/enilnets_amd.h``).
"""

from .compression import (QUANTIZABLE, ActivationCalibrator, compute_scale, dequantize,
                          fake_quantize, quant_range, quantization_error, quantize,
                          quantize_tensor, quantize_weights, remove_activation_quantization)
from .device import DeviceArray
from .nn import Forward, Model

__version__ = "0.1.0"

__all__ = [
    "quantize_weights", "ActivationCalibrator", "quantize_tensor", "fake_quantize",
    "quantize", "dequantize", "compute_scale", "quant_range", "quantization_error",
    "remove_activation_quantization", "QUANTIZABLE", "Forward", "Model", "DeviceArray",
]
