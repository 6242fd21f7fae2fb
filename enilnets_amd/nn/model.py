"""A minimal model holding layer dicts in the reference's schema.

Enilnets' ``NeuralNet`` keeps its network as ``self.layers``, a list of plain
dicts (``Enilnets/nn/layers.py:26-27`` for Dense:
``{"type": "dense", "weights": (n_out, n_in), "bias": (n_out,),
"activation", "use_bias", "activation_params"}``).  Every function of this
package accepts any object with such a ``layers`` list; ``Model`` is a small
stand-in used by the tests and the benchmark, whose ``Forward`` is the GPU
one.
"""

import copy
from typing import Any, Dict, List, Optional

import numpy as np


class Model:
    def __init__(self) -> None:
        self.layers: List[Dict[str, Any]] = []
        self.outputs: List[Any] = []
        self.pre_activations: List[Any] = []

    def add_dense(self, weights: np.ndarray, bias: Optional[np.ndarray] = None,
                  activation: str = "relu",
                  activation_params: Optional[Dict[str, Any]] = None) -> Dict[str, Any]:
        """Append a Dense layer with the given ``(n_out, n_in)`` weights."""
        w = np.asarray(weights)
        b = np.zeros(w.shape[0], w.dtype) if bias is None else np.asarray(bias)
        layer = {"type": "dense", "weights": w, "bias": b, "activation": activation,
                 "use_bias": bias is not None, "activation_params": activation_params or {}}
        self.layers.append(layer)
        return layer

    def Forward(self, inputs: Any, training: bool = False, dropout_rate: float = 0.0,
                variant: str = "fp32") -> np.ndarray:
        from .forward import Forward
        return Forward(self, inputs, training, dropout_rate, variant)

    predict = Forward

    def copy(self) -> "Model":
        return copy.deepcopy(self)
