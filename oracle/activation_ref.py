"""CPU oracle of SiLU-and-Mul — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, as the checker; the product path never calls it.

Restates the reference contract (vllm_rlt/kernels/activation.py:20-33,
tests/test_activation.py:55-72): ``F.silu(gate) * up`` with the SiLU rounded to
the storage dtype before the multiply. The SiLU value is computed in float64
and rounded the way torch converts float64 to a storage dtype: to float32
first, then to the dtype (nearest-even both times). The product of two dtype
values is exact in float64 and is rounded the same way.

Pinning (tests/test_oracle.py): the known values of
tests/test_activation.py:49-53, torch's float64 ``F.silu`` (library routine),
the identity silu(x) - silu(-x) = x, and torch's own double -> dtype
conversion over every bf16 / f16 bit pattern.
"""

from __future__ import annotations

import numpy as np

from oracle.paged_ref import round_to


def silu_f64(x: np.ndarray) -> np.ndarray:
    """silu(x) = x * sigmoid(x) in float64, overflow-free on both signs."""
    with np.errstate(over="ignore", invalid="ignore"):
        x = np.asarray(x, dtype=np.float64)
        pos = x / (1.0 + np.exp(-np.maximum(x, 0.0)))
        t = np.exp(np.minimum(x, 0.0))
        neg = x * t / (1.0 + t)
    return np.where(x >= 0.0, pos, neg)


def _to_dtype(x64: np.ndarray, dtype: str) -> np.ndarray:
    with np.errstate(over="ignore", invalid="ignore"):
        return round_to(x64.astype(np.float32), dtype)


def silu_and_mul(gate: np.ndarray, up: np.ndarray, dtype: str) -> np.ndarray:
    """Result values (float32 array holding dtype-representable values).

    ``gate`` and ``up`` are float32 arrays already holding dtype values."""
    act = _to_dtype(silu_f64(gate), dtype)
    with np.errstate(over="ignore", invalid="ignore"):
        prod = act.astype(np.float64) * np.asarray(up, dtype=np.float64)
    return _to_dtype(prod, dtype)
