"""Quantized-path execution: device-resident Dense layers and the drop-in
``Forward``."""

from .dense import (dense_w8, dense_w8a8, gemm_w8a8, quantize_rows_i8,
                    quantize_weight_rows)
from .forward import Forward
from .io import LoadInt8, SaveInt8
from .model import Model
from .weights import Int8Weights, int8_weights

__all__ = ["Forward", "Model", "SaveInt8", "LoadInt8", "Int8Weights", "int8_weights", "dense_w8", "dense_w8a8",
           "gemm_w8a8", "quantize_rows_i8", "quantize_weight_rows"]
