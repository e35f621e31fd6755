"""Oracle restatement of the structured-state transform.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

- ``transform_delta_state``: ``cb/architectures/qwen35.py:52-61``, the
  recurrent (DeltaNet) memory mapped as ``key_basis^T @ source_state @
  value_basis`` over broadcast batch dimensions, in float64 numpy. Parity
  pinned by the reference test ``tests/test_architectures.py:100-111``
  (bilinear read-out ``q @ mapped == einsum(q, a, state, b)`` for rectangular
  bases, restated) and by a brute-force triple loop on tiny inputs.
"""

from __future__ import annotations

import numpy as np


def transform_delta_state(source_state, key_basis, value_basis) -> np.ndarray:
    """``A^T U B`` in float64 (inputs are array-likes, e.g. CPU tensors)."""
    u = np.asarray(source_state, dtype=np.float64)
    a = np.asarray(key_basis, dtype=np.float64)
    b = np.asarray(value_basis, dtype=np.float64)
    if min(u.ndim, a.ndim, b.ndim) < 2:
        raise ValueError("Delta state and basis tensors must be matrix-valued")
    if u.shape[-2] != a.shape[-2] or u.shape[-1] != b.shape[-2]:
        raise ValueError("Source state dimensions do not match the key/value bases")
    return np.swapaxes(a, -2, -1) @ u @ b


def transform_delta_state_loops(u, a, b) -> np.ndarray:
    """The same product as explicit sums (one unbatched matrix triple)."""
    u, a, b = (np.asarray(x, dtype=np.float64) for x in (u, a, b))
    k, v = u.shape
    kp, vp = a.shape[1], b.shape[1]
    out = np.zeros((kp, vp))
    for i in range(kp):
        for j in range(vp):
            out[i, j] = sum(a[r, i] * u[r, c] * b[c, j] for r in range(k) for c in range(v))
    return out
