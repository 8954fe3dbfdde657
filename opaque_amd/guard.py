"""Host-side constants of the clip-scale guard.

The reference shrinks every clip ratio so that the bound still holds after
the norm reduction, the downcast of the scale and the per-element multiply
(``opaque-engine/.../clipping/_pytree.py:81-142,156-221``):

    roundoff = (u_acc + (max(n_leaves, 1) + n_reduction) * u_sq) / 2
    rel      = 1 - 2 * (eps_store / 2 + roundoff)
    abs      = smallest_normal_store * eps_store
    scale    = ratio * rel - abs

with u = eps/2 of the accumulation dtype (float32 for bf16/fp16/fp32
leaves) and of the fp64 cross-leaf sum, and ``n_reduction`` the worst-case
sequential additions of the widest leaf's two-stage (2048-wide) reduction.
These are evaluated here in Python floats exactly as the reference
evaluates them; the device applies ``ratio * rel - abs`` in fp64.
"""

from __future__ import annotations

import math
from collections.abc import Iterable

import torch

REDUCTION_BLOCK = 2048
BLOCKED_REDUCTION_MIN = 4096
SQ_ACCUM_DTYPE = torch.float64


def blocked_reduction_terms(n: int) -> int:
    return REDUCTION_BLOCK + (n + REDUCTION_BLOCK - 1) // REDUCTION_BLOCK


def reduction_terms(leaf_numels: Iterable[int]) -> int:
    widest = 0
    for n in leaf_numels:
        widest = max(widest, int(n))
    if widest <= 1:
        return 0
    if widest > BLOCKED_REDUCTION_MIN:
        return blocked_reduction_terms(widest)
    return widest


def accumulation_dtype(leaf_dtypes: Iterable[torch.dtype], compute_dtype: torch.dtype | None) -> torch.dtype:
    """Dtype of the per-element squares (``_resolve_compute_dtype_for_reduction``)."""
    if compute_dtype is not None:
        if not compute_dtype.is_floating_point:
            raise TypeError(
                f"compute_dtype must be a real floating-point dtype, got {compute_dtype!r}."
            )
        return compute_dtype
    acc = torch.float32
    for dt in leaf_dtypes:
        if not (dt.is_floating_point or dt.is_complex):
            continue
        real = torch.empty((), dtype=dt).real.dtype if dt.is_complex else dt
        promoted = torch.float32 if real in (torch.float16, torch.bfloat16) else real
        acc = torch.promote_types(acc, promoted)
    return acc


def norm_roundoff(acc_dtype: torch.dtype, n_leaves: int, n_reduction: int,
                  sq_dtype: torch.dtype = SQ_ACCUM_DTYPE) -> float:
    u_acc = torch.finfo(acc_dtype).eps / 2.0 if acc_dtype.is_floating_point else 0.0
    u_sq = torch.finfo(sq_dtype).eps / 2.0 if sq_dtype.is_floating_point else 0.0
    return (u_acc + (max(n_leaves, 1) + n_reduction) * u_sq) / 2.0


def guard_constants(storage_dtype: torch.dtype, roundoff: float) -> tuple[float, float]:
    """(rel, abs) such that the stored scale is ``ratio * rel - abs``."""
    if not (storage_dtype.is_floating_point or storage_dtype.is_complex):
        return 1.0, 0.0
    store = torch.finfo(storage_dtype)
    return 1.0 - 2.0 * (store.eps / 2.0 + roundoff), store.smallest_normal * store.eps


def leaf_guards(leaf_shapes: list[tuple[int, ...]], leaf_dtypes: list[torch.dtype],
                compute_dtype: torch.dtype | None = None) -> tuple[torch.dtype, float]:
    """(accumulation dtype, roundoff) for one per-example gradient pytree."""
    acc = accumulation_dtype(leaf_dtypes, compute_dtype)
    n_red = reduction_terms(math.prod(s) for s in leaf_shapes)
    return acc, norm_roundoff(acc, len(leaf_shapes), n_red)


__all__ = [
    "accumulation_dtype",
    "blocked_reduction_terms",
    "guard_constants",
    "leaf_guards",
    "norm_roundoff",
    "reduction_terms",
]
