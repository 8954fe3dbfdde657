"""DP wrapper types that carry sensitivity metadata between clip and noise.

Same names, fields and arithmetic rules as ``opaque-engine/.../engine/types.py``
(PerGroup :70-153, ClippedPytree :247-381, NoisedPytree :384-401, paired
outputs :409-445, factories :453-465) so code written against the reference
keeps working.
"""

from __future__ import annotations

import math
from abc import ABC
from dataclasses import dataclass, replace
from numbers import Real
from types import MappingProxyType
from typing import Any, Literal, NamedTuple

import torch

from opaque_amd.pytree import ParamPath, param_path, tree_map

TensorPytree = Any
MaxNorm = Any
NoiseStddev = Any


@dataclass(frozen=True)
class PerGroup:
    """Per-group scalar values with a resolved leaf-path -> group mapping."""

    groups: Any  # Mapping[ParamPath | str, str]
    values: Any  # Mapping[str, float]

    def __post_init__(self) -> None:
        norm = {param_path(k): g for k, g in self.groups.items()}
        object.__setattr__(self, "groups", MappingProxyType(norm))
        object.__setattr__(self, "values", MappingProxyType(dict(self.values)))

    @property
    def effective(self) -> float:
        """sqrt(sum v^2): the scalar value used for accounting."""
        return math.sqrt(sum(v**2 for v in self.values.values()))

    def __rmul__(self, scalar: float) -> PerGroup:
        return PerGroup(self.groups, {k: scalar * v for k, v in self.values.items()})

    def __mul__(self, other: float | PerGroup) -> PerGroup:
        if isinstance(other, PerGroup):
            if other.groups != self.groups:
                raise ValueError(
                    "PerGroup × PerGroup requires identical group mappings; "
                    f"got groups with {len(self.groups)} vs {len(other.groups)} parameter assignments."
                )
            if set(other.values) != set(self.values):
                raise ValueError(
                    "PerGroup × PerGroup requires identical group sets; "
                    f"got {sorted(self.values)} vs {sorted(other.values)}."
                )
            return PerGroup(self.groups, {k: v * other.values[k] for k, v in self.values.items()})
        return PerGroup(self.groups, {k: v * other for k, v in self.values.items()})

    def __truediv__(self, scalar: float) -> PerGroup:
        return PerGroup(self.groups, {k: v / scalar for k, v in self.values.items()})

    def for_path(self, path: ParamPath | str) -> float:
        return self.values[self.groups[param_path(path)]]


class ClipState(ABC):  # noqa: B024 - marker base
    """Base class of clipping states."""


class NoiseState(ABC):  # noqa: B024 - marker base
    """Base class of noise states (``_step_counter``, ``_rng_key``)."""

    _step_counter: int
    _rng_key: Any


def _public_scalar(scalar: Any, *, op: str) -> float:
    if isinstance(scalar, bool) or not isinstance(scalar, Real):
        raise TypeError(
            f"{op} only supports public real-number scalars. "
            "Operate on `.pytree` and reconstruct the clipped value with an "
            "explicit max_norm when the clipped interpretation is unclear."
        )
    return float(scalar)


def _unsupported(op: str) -> str:
    return (
        f"ClippedPytree {op} does not preserve DP max_norm semantics "
        "automatically. Operate on `.pytree` and reconstruct the clipped "
        "value with an explicit max_norm."
    )


def _apply_method(pytree: Any, method: str, *args: Any, **kwargs: Any) -> Any:
    return tree_map(
        lambda x: getattr(x, method)(*args, **kwargs) if isinstance(x, torch.Tensor) else x, pytree
    )


@dataclass(frozen=True)
class ClippedPytree:
    """A pytree whose per-record contribution has L2 norm at most ``max_norm``."""

    pytree: Any
    max_norm: MaxNorm

    @property
    def sensitivity(self) -> float:
        eff = getattr(self.max_norm, "effective", None)
        return float(eff) if eff is not None else float(self.max_norm)

    def noise_stddev_for(
        self, *, noise_multiplier: float, allocation: Literal["isotropic", "optimal"] = "optimal"
    ) -> float | PerGroup:
        if noise_multiplier < 0:
            raise ValueError(f"noise_multiplier must be non-negative, got {noise_multiplier}")
        if allocation not in ("isotropic", "optimal"):
            raise ValueError(f"allocation must be 'isotropic' or 'optimal', got {allocation!r}.")
        if isinstance(self.max_norm, PerGroup):
            if allocation == "isotropic":
                return noise_multiplier * self.max_norm.effective
            from opaque_amd.noise_allocation import per_group_noise_stddev

            return per_group_noise_stddev(self.max_norm, noise_multiplier)
        return noise_multiplier * float(self.max_norm)

    def _scaled(self, s: float) -> ClippedPytree:
        return replace(
            self,
            pytree=tree_map(lambda x: x * s if isinstance(x, torch.Tensor) else x, self.pytree),
            max_norm=abs(s) * self.max_norm,
        )

    def __mul__(self, scalar: Any) -> ClippedPytree:
        return self._scaled(_public_scalar(scalar, op="ClippedPytree *"))

    def __rmul__(self, scalar: Any) -> ClippedPytree:
        return self._scaled(_public_scalar(scalar, op="* ClippedPytree"))

    def __truediv__(self, scalar: Any) -> ClippedPytree:
        s = _public_scalar(scalar, op="ClippedPytree /")
        if s == 0.0:
            raise ZeroDivisionError("ClippedPytree division by zero")
        return self._scaled(1.0 / s)

    def __rtruediv__(self, scalar: Any) -> ClippedPytree:
        raise TypeError(_unsupported("reverse division"))

    def __neg__(self) -> ClippedPytree:
        return self._scaled(-1.0)

    def __add__(self, other: Any) -> ClippedPytree:
        raise TypeError(_unsupported("addition"))

    __radd__ = __add__

    def __sub__(self, other: Any) -> ClippedPytree:
        raise TypeError(_unsupported("subtraction"))

    __rsub__ = __sub__

    def __pow__(self, exponent: Any) -> ClippedPytree:
        raise TypeError(_unsupported("power"))

    def clone(self) -> ClippedPytree:
        return replace(self, pytree=_apply_method(self.pytree, "clone"))

    def detach(self) -> ClippedPytree:
        return replace(self, pytree=_apply_method(self.pytree, "detach"))

    def to(self, *args: Any, **kwargs: Any) -> ClippedPytree:
        return replace(self, pytree=_apply_method(self.pytree, "to", *args, **kwargs))


@dataclass(frozen=True)
class NoisedPytree(ClippedPytree):
    """A privatised pytree; ``noise_stddev`` records the noise actually added."""

    noise_stddev: NoiseStddev = None

    def _scaled(self, s: float) -> NoisedPytree:
        return replace(
            self,
            pytree=tree_map(lambda x: x * s if isinstance(x, torch.Tensor) else x, self.pytree),
            max_norm=abs(s) * self.max_norm,
            noise_stddev=None if self.noise_stddev is None else abs(s) * self.noise_stddev,
        )


class SecondMomentClippingOutput(NamedTuple):
    """Paired pre-noise streams: clipped sum and clipped sum of squares."""

    grads: ClippedPytree
    squared_grads: ClippedPytree


class SecondMomentNoiseOutput(NamedTuple):
    noisy_grads: NoisedPytree
    noisy_squared_grads: NoisedPytree


def clipped(pytree: Any, *, max_norm: MaxNorm) -> ClippedPytree:
    return ClippedPytree(pytree=pytree, max_norm=max_norm)


def noised(pytree: Any, *, max_norm: MaxNorm, noise_stddev: NoiseStddev) -> NoisedPytree:
    return NoisedPytree(pytree=pytree, max_norm=max_norm, noise_stddev=noise_stddev)


__all__ = [
    "ClipState",
    "ClippedPytree",
    "MaxNorm",
    "NoiseState",
    "NoiseStddev",
    "NoisedPytree",
    "ParamPath",
    "PerGroup",
    "SecondMomentClippingOutput",
    "SecondMomentNoiseOutput",
    "TensorPytree",
    "clipped",
    "noised",
]
