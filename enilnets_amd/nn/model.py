"""A minimal model holding layer dicts in the reference's schema.

Enilnets' ``NeuralNet`` keeps its network as ``self.layers``, a list of plain
dicts (``Enilnets/nn/layers.py:26-27`` for Dense:
``{"type": "dense", "weights": (n_out, n_in), "bias": (n_out,),
"activation", "use_bias", "activation_params"}``).  Every function of this
package accepts any object with such a ``layers`` list; ``Model`` is a small
stand-in used by the tests and the benchmark, whose ``Forward`` is the GPU
one.  Its builders take explicit weights (the reference's draw them from
its initialisers) and produce the reference's dict layouts.
"""

import copy
from typing import Any, Dict, List, Optional

import numpy as np


class Model:
    def __init__(self) -> None:
        self.layers: List[Dict[str, Any]] = []
        self._residual_stack: List[int] = []
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

    def add_layernorm(self, width: int, epsilon: float = 1e-5) -> Dict[str, Any]:
        """LayerNorm over the last axis (``layers.py:181-194``): gamma ones,
        beta zeros."""
        layer = {"type": "layernorm", "normalized_shape": width, "epsilon": epsilon,
                 "gamma": np.ones(width, np.float32), "beta": np.zeros(width, np.float32)}
        self.layers.append(layer)
        return layer

    def add_residual_start(self) -> Dict[str, Any]:
        """Marks the input saved for the matching ``add_residual_end``
        (``layers.py:609-623``)."""
        self._residual_stack.append(len(self.layers))
        layer = {"type": "residual_save"}
        self.layers.append(layer)
        return layer

    def add_residual_end(self) -> Dict[str, Any]:
        """``x = x + saved_x`` (``layers.py:625-632``)."""
        if not self._residual_stack:
            raise ValueError("add_residual_end() called without a matching add_residual_start()")
        layer = {"type": "residual_add", "save_index": self._residual_stack.pop()}
        self.layers.append(layer)
        return layer

    def add_multihead_attention(self, wq: np.ndarray, wk: np.ndarray, wv: np.ndarray,
                                wo: np.ndarray, num_heads: int,
                                num_kv_heads: Optional[int] = None, causal: bool = False,
                                window_size: Optional[int] = None,
                                biases: Optional[Dict[str, np.ndarray]] = None) -> Dict[str, Any]:
        """Softmax self-attention with the given ``(out, in)`` projection
        weights, in the dict layout of ``layers.py:328-349``; biases default
        to zeros."""
        embed = wq.shape[1]
        head_dim = embed // num_heads
        kv_heads = num_heads if num_kv_heads is None else num_kv_heads
        biases = biases or {}
        layer = {"type": "multihead_attention", "embed_dim": embed, "num_heads": num_heads,
                 "num_kv_heads": kv_heads, "head_dim": head_dim, "dropout": 0.0,
                 "causal": causal, "window_size": window_size, "attention_kernel": "softmax",
                 "sparse_pattern": None, "tiled_block_size": None,
                 "positional_scheme": "absolute"}
        for name, w in (("q", wq), ("k", wk), ("v", wv), ("o", wo)):
            w = np.asarray(w)
            layer["W" + name] = w
            layer["b" + name] = np.asarray(biases.get("b" + name, np.zeros(w.shape[0], w.dtype)))
        self.layers.append(layer)
        return layer

    def add_moe(self, w1: np.ndarray, w2: np.ndarray, wr: np.ndarray, top_k: int = 1,
                activation: str = "gelu", b1: Optional[np.ndarray] = None,
                b2: Optional[np.ndarray] = None,
                br: Optional[np.ndarray] = None) -> Dict[str, Any]:
        """Mixture of experts with stacked ``W1 (E, H, D)``, ``W2 (E, D, H)``
        and router ``Wr (E, D)``, in the dict layout of ``layers.py:387-398``;
        biases default to zeros."""
        n_exp, hidden, embed = np.shape(w1)
        layer = {"type": "moe", "embed_dim": embed, "num_experts": n_exp, "hidden_dim": hidden,
                 "top_k": top_k, "activation": activation, "aux_loss_weight": 0.01,
                 "W1": np.asarray(w1), "W2": np.asarray(w2), "Wr": np.asarray(wr),
                 "b1": np.zeros((n_exp, hidden), np.float32) if b1 is None else np.asarray(b1),
                 "b2": np.zeros((n_exp, embed), np.float32) if b2 is None else np.asarray(b2),
                 "br": np.zeros(n_exp, np.float32) if br is None else np.asarray(br)}
        self.layers.append(layer)
        return layer

    def Forward(self, inputs: Any, training: bool = False, dropout_rate: float = 0.0,
                variant: str = "fp32") -> np.ndarray:
        from .forward import Forward
        return Forward(self, inputs, training, dropout_rate, variant)

    predict = Forward

    def copy(self) -> "Model":
        return copy.deepcopy(self)
