"""Per-group and paired-stream noise standard deviations.

Formulas of ``opaque-engine/.../engine/noise_allocation.py``: single stream
sigma_g = nm * sqrt(C_g * sum_h C_h) (:33-95); paired release with
S = sum_h (D1_h + D2_h), sigma = nm * sqrt(D * S) per stream (:136-232);
fold-in tags 1 and 2 namespace the paired streams (:29-30).
"""

from __future__ import annotations

import math

from opaque_amd.types import ClippedPytree, PerGroup, SecondMomentClippingOutput

PAIRED_FIRST_STREAM_FOLD = 1
PAIRED_SECOND_STREAM_FOLD = 2


def per_group_noise_stddev(max_norm: PerGroup, noise_multiplier: float) -> PerGroup:
    if not isinstance(max_norm, PerGroup):
        raise TypeError(
            f"per_group_noise_stddev requires a PerGroup max_norm, got {type(max_norm).__name__}."
        )
    if noise_multiplier < 0:
        raise ValueError(f"noise_multiplier must be non-negative, got {noise_multiplier}")
    for name, v in max_norm.values.items():
        if v < 0:
            raise ValueError(f"per-group bounds must be non-negative, got {v} for group '{name}'.")
    if noise_multiplier == 0.0:
        return PerGroup(max_norm.groups, dict.fromkeys(max_norm.values, 0.0))
    total = sum(max_norm.values.values())
    return PerGroup(
        max_norm.groups,
        {k: noise_multiplier * math.sqrt(c * total) for k, c in max_norm.values.items()},
    )


def _check_sensitivity(value: float | PerGroup, *, label: str) -> None:
    if isinstance(value, PerGroup):
        for name, v in value.values.items():
            if v < 0:
                raise ValueError(
                    f"{label} per-group bounds must be non-negative, got {v} for group '{name}'."
                )
    else:
        if not isinstance(value, (int, float)):
            raise TypeError(f"{label} must be float or PerGroup, got {type(value).__name__}.")
        if value < 0:
            raise ValueError(f"{label} must be non-negative, got {value}.")


def _total(value: float | PerGroup) -> float:
    return float(sum(value.values.values())) if isinstance(value, PerGroup) else float(value)


def _sigma(value: float | PerGroup, total: float, nm: float) -> float | PerGroup:
    if isinstance(value, PerGroup):
        return PerGroup(value.groups, {k: nm * math.sqrt(v * total) for k, v in value.values.items()})
    return nm * math.sqrt(float(value) * total)


def paired_noise_stddevs(
    noise_multiplier: float, *, first: float | PerGroup, second: float | PerGroup
) -> tuple[float | PerGroup, float | PerGroup]:
    if isinstance(first, PerGroup) != isinstance(second, PerGroup):
        raise TypeError(
            "paired_noise_stddevs requires both streams to have the same kind; "
            f"got first={type(first).__name__}, second={type(second).__name__}."
        )
    if noise_multiplier < 0:
        raise ValueError(f"noise_multiplier must be non-negative, got {noise_multiplier}")
    _check_sensitivity(first, label="first")
    _check_sensitivity(second, label="second")
    if isinstance(first, PerGroup):
        if first.groups != second.groups:
            raise ValueError(
                "paired_noise_stddevs requires identical group mappings on both streams; got "
                f"{len(first.groups)} vs {len(second.groups)} parameter assignments."
            )
        if set(first.values) != set(second.values):
            raise ValueError(
                "paired_noise_stddevs requires identical group sets on both streams; got "
                f"{sorted(first.values)} vs {sorted(second.values)}."
            )
    total = _total(first) + _total(second)
    return _sigma(first, total, noise_multiplier), _sigma(second, total, noise_multiplier)


def resolve_paired_clipped(clipped_input: SecondMomentClippingOutput, *, noise_multiplier: float):
    first, second = clipped_input.grads, clipped_input.squared_grads
    if not isinstance(first, ClippedPytree):
        raise TypeError("SecondMomentClippingOutput.grads must be a ClippedPytree.")
    if not isinstance(second, ClippedPytree):
        raise TypeError("SecondMomentClippingOutput.squared_grads must be a ClippedPytree.")
    s1, s2 = paired_noise_stddevs(noise_multiplier, first=first.max_norm, second=second.max_norm)
    return first, second, s1, s2


__all__ = [
    "PAIRED_FIRST_STREAM_FOLD",
    "PAIRED_SECOND_STREAM_FOLD",
    "paired_noise_stddevs",
    "per_group_noise_stddev",
    "resolve_paired_clipped",
]
