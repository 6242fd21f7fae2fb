"""Dense weight initialisation with the reference's layout and random draws.

Restates ``Enilnets/nn/weight_init.py:11-46`` (``init_weights``): weights
``(n_out, n_in)`` and a zero bias ``(n_out,)``, float32, drawn from NumPy's
global random state in the same calls, so a seeded run gives the same
weights as the reference.  Host-side set-up, not part of the GPU path.
"""

from typing import Any, Optional, Tuple

import numpy as np

#: ``Enilnets/core/constants.py:67``.
NORMAL_INIT_STD = 0.1


def init_weights(n_in: int, n_out: int, method: str = "xavier_uniform",
                 std: Optional[float] = None, dtype: Any = np.float32) -> Tuple[np.ndarray, np.ndarray]:
    """``(weights (n_out, n_in), bias (n_out,))``; ValueError for an unknown method."""
    shape = (n_out, n_in)
    if method == "xavier_uniform":
        limit = np.sqrt(6 / (n_in + n_out))
        w = np.random.uniform(-limit, limit, shape).astype(dtype)
    elif method == "xavier_normal":
        w = np.random.normal(0, np.sqrt(2 / (n_in + n_out)), shape).astype(dtype)
    elif method == "he_uniform":
        limit = np.sqrt(6 / n_in)
        w = np.random.uniform(-limit, limit, shape).astype(dtype)
    elif method == "he_normal":
        w = np.random.normal(0, np.sqrt(2 / n_in), shape).astype(dtype)
    elif method == "normal":
        w = np.random.normal(0, NORMAL_INIT_STD if std is None else std, shape).astype(dtype)
    elif method == "orthogonal":
        g = np.random.normal(0, 1, shape).astype(dtype)
        u, _, vt = np.linalg.svd(g, full_matrices=False)
        w = u @ vt
    elif method == "zeros":
        w = np.zeros(shape, dtype=dtype)
    elif method == "ones":
        w = np.ones(shape, dtype=dtype)
    else:
        raise ValueError(f"Unknown initialization method: {method}")
    return w, np.zeros(n_out, dtype=dtype)
