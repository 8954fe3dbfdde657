"""``adaptive_clipped_grad``: quantile-tracking clip threshold (Andrew et al., 2021).

Same factory, state, aux type, validation and update rule as
``opaque-dpsgd/.../clipping/_adaptive.py:25-642``: each step clips at the
current threshold C (through the same native kernels as ``clipped_grad``),
counts the clipped examples, adds Gaussian noise of std
``fraction_noise_std`` to the clipped fraction (drawn from a CPU generator
seeded by ``fold_in(key, step)``, per group ``fold_in(fold_in(key, step), i)``
in sorted group-name order) and moves the threshold geometrically:
C <- clamp(C * exp(lr * (rate_noisy - target_quantile)), min, max).
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

import torch
from torch.autograd.profiler import record_function

from opaque_amd.clipping import (
    ClippedGradAux,
    ClippingStats,
    _ClipEngine,
    _identity,
    _to_tuple,
    _validate_static_args,
    _zero_grads_like,
    batch_size_from_args,
)
from opaque_amd.random import RngKey, fold_in, generator_from_key
from opaque_amd.types import ClipState, PerGroup, SecondMomentClippingOutput, clipped

_DEFAULT_FRACTION_NOISE_STD = 0.05


@dataclass(frozen=True)
class AdaptiveClippedGradAux(ClippedGradAux):
    """``ClippedGradAux`` of an adaptive-threshold step."""


@dataclass(frozen=True)
class AdaptiveClipState(ClipState):
    """Threshold used this step, threshold for the next, step counter, config and counts."""

    _current_clipping_norm: float | PerGroup
    _next_clipping_norm: float | PerGroup
    _step: int
    _rng_key: RngKey
    _fraction_noise_std: float
    _learning_rate: float
    _target_quantile: float
    _clipping_norm_min: float
    _clipping_norm_max: float
    _num_clipped: float | dict[str, float]
    _batch_size: float

    def __post_init__(self) -> None:
        if isinstance(self._next_clipping_norm, PerGroup):
            for name, val in self._next_clipping_norm.values.items():
                if val <= 0:
                    raise ValueError(
                        f"next_clipping_norm must be positive for all groups, got {val} for group '{name}'"
                    )
        elif self._next_clipping_norm <= 0:
            raise ValueError(f"next_clipping_norm must be positive, got {self._next_clipping_norm}")
        if self._fraction_noise_std <= 0:
            raise ValueError(f"fraction_noise_std must be > 0, got {self._fraction_noise_std}")


def _sample_noisy_clipping_rate(clipping_rate: float, *, key: RngKey, step: int,
                                fraction_noise_std: float) -> float:
    """rate + N(0, std^2) from a CPU generator seeded by fold_in(key, step) (_adaptive.py:100-110)."""
    generator = generator_from_key(fold_in(key, step))
    return clipping_rate + torch.randn(1, generator=generator).item() * fraction_noise_std


def _adaptive_clipping_norm_update(*, base_clipping_norm: float, noisy_clipping_rate: float,
                                   target_quantile: float, learning_rate: float,
                                   clipping_norm_min: float, clipping_norm_max: float) -> float:
    """clamp(C * exp(lr * (rate - target)), min, max), the factor evaluated as a float32 tensor."""
    factor = torch.exp(torch.tensor(learning_rate * (noisy_clipping_rate - target_quantile))).item()
    return float(max(clipping_norm_min, min(clipping_norm_max, base_clipping_norm * factor)))


def adaptive_clipped_grad(
    loss_fn: Callable,
    argnums: int | tuple[int, ...] = 0,
    has_aux: bool = False,
    *,
    initial_clipping_norm: float | PerGroup = 0.1,
    target_quantile: float = 0.5,
    learning_rate: float = 0.2,
    clipping_norm_min: float = 0.01,
    clipping_norm_max: float = 100.0,
    fraction_noise_std: float = _DEFAULT_FRACTION_NOISE_STD,
    key: RngKey,
    return_aux: bool = False,
    return_stats: bool = False,
    pre_clipping_transform: Callable = _identity,
    **clipped_grad_kwargs: Any,
) -> tuple[Callable, AdaptiveClipState]:
    """Clipped gradients whose threshold tracks ``target_quantile`` of the norms (``_adaptive.py:132-642``)."""
    if return_aux and return_stats:
        raise ValueError("return_stats cannot be combined with return_aux=True")
    if isinstance(initial_clipping_norm, PerGroup):
        for name, val in initial_clipping_norm.values.items():
            if val <= 0:
                raise ValueError(
                    f"initial_clipping_norm must be positive for all groups, got {val} for group '{name}'"
                )
    elif initial_clipping_norm <= 0:
        raise ValueError(f"initial_clipping_norm must be positive, got {initial_clipping_norm}")
    if not 0 < target_quantile < 1:
        raise ValueError(f"target_quantile must be in (0, 1), got {target_quantile}")
    if learning_rate <= 0:
        raise ValueError(f"learning_rate must be positive, got {learning_rate}")
    if clipping_norm_min <= 0:
        raise ValueError(f"clipping_norm_min must be positive, got {clipping_norm_min}")
    if clipping_norm_max <= clipping_norm_min:
        raise ValueError(
            f"clipping_norm_max ({clipping_norm_max}) must be > clipping_norm_min ({clipping_norm_min})"
        )
    if fraction_noise_std <= 0:
        raise ValueError(f"fraction_noise_std must be positive, got {fraction_noise_std}")

    argnums_t = _to_tuple(argnums)
    batch_raw = clipped_grad_kwargs.pop("batch_argnums", 1)
    batch_t = _to_tuple(batch_raw)
    normalize_by = clipped_grad_kwargs.pop("normalize_by", 1.0)
    second_moment = bool(clipped_grad_kwargs.pop("second_moment", False))
    microbatch_size = clipped_grad_kwargs.pop("microbatch_size", None)
    dtype = clipped_grad_kwargs.pop("dtype", None)
    compute_dtype = clipped_grad_kwargs.pop("compute_dtype", None)
    if clipped_grad_kwargs:
        raise TypeError(f"unexpected keyword arguments: {sorted(clipped_grad_kwargs)}")
    _validate_static_args(argnums, batch_raw, normalize_by)
    is_per_group = isinstance(initial_clipping_norm, PerGroup)
    config = dict(target_quantile=target_quantile, learning_rate=learning_rate,
                  clipping_norm_min=clipping_norm_min, clipping_norm_max=clipping_norm_max,
                  fraction_noise_std=fraction_noise_std)
    engine = _ClipEngine(
        loss_fn, argnums_t, argnums, has_aux, clipping_norm=initial_clipping_norm, autos=False, gamma=0.0,
        normalize_by=normalize_by, batch_argnums=batch_t, want_aux=return_aux, want_stats=not return_aux,
        second_moment=second_moment, pre_clipping_transform=pre_clipping_transform,
        microbatch_size=microbatch_size, dtype=dtype, compute_dtype=compute_dtype, scale_fn=None,
    )

    def _empty_counts():
        return dict.fromkeys(initial_clipping_norm.values, 0.0) if is_per_group else 0.0

    def _next_state(state: AdaptiveClipState, nxt, num_clipped, batch_size: float) -> AdaptiveClipState:
        return AdaptiveClipState(
            _current_clipping_norm=state._next_clipping_norm, _next_clipping_norm=nxt, _step=state._step + 1,
            _rng_key=state._rng_key, _fraction_noise_std=config["fraction_noise_std"],
            _learning_rate=config["learning_rate"], _target_quantile=config["target_quantile"],
            _clipping_norm_min=config["clipping_norm_min"], _clipping_norm_max=config["clipping_norm_max"],
            _num_clipped=num_clipped, _batch_size=batch_size,
        )

    def _update(threshold: float, rate: float, generator_key: RngKey) -> float:
        noise = torch.randn(1, generator=generator_from_key(generator_key)).item() * config["fraction_noise_std"]
        return _adaptive_clipping_norm_update(
            base_clipping_norm=threshold, noisy_clipping_rate=rate + noise,
            target_quantile=config["target_quantile"], learning_rate=config["learning_rate"],
            clipping_norm_min=config["clipping_norm_min"], clipping_norm_max=config["clipping_norm_max"])

    def grad_fn(*args, state: AdaptiveClipState, **kwargs):
        with record_function("opaque::adaptive_clipped_grad"):
            C = state._next_clipping_norm
            max_norm = C / normalize_by
            if batch_size_from_args(args, batch_t) == 0:
                grads: Any = clipped(_zero_grads_like(args, argnums_t), max_norm=max_norm)
                if second_moment:
                    grads = SecondMomentClippingOutput(
                        grads=grads,
                        squared_grads=clipped(_zero_grads_like(args, argnums_t), max_norm=(C * C) / normalize_by))
                new_state = _next_state(state, C, _empty_counts(), 0.0)
                if return_aux:
                    empty = torch.empty(0)
                    return (grads, AdaptiveClippedGradAux(loss_values=empty, grad_norms=empty,
                                                          clipped_grad_norms=empty, loss_aux=None,
                                                          clipping_rate=0.0)), new_state
                if return_stats:
                    zero = _empty_counts()
                    return (grads, ClippingStats(num_clipped=zero, clipping_rate=zero if is_per_group else 0.0,
                                                 batch_size=0)), new_state
                return grads, new_state

            engine.clipping_norm = C
            grads, info = engine(args, kwargs)
            aux = info if return_aux else None
            stats = None if return_aux else info
            batch_size = aux.batch_size if aux is not None else stats.batch_size
            if is_per_group:
                new_values: dict[str, float] = {}
                counts: dict[str, float] = {}
                for i, name in enumerate(sorted(C.values.keys())):
                    threshold = C.values[name]
                    if stats is not None:
                        nc = stats.num_clipped.get(name, 0.0)
                        rate = stats.clipping_rate.get(name, 0.0)
                    else:
                        nc = float((aux.group_norms[name] > threshold).sum().item())
                        rate = nc / max(1.0, float(batch_size))
                    counts[name] = nc
                    new_values[name] = _update(threshold, rate, fold_in(fold_in(state._rng_key, state._step), i))
                nxt: float | PerGroup = PerGroup(groups=C.groups, values=new_values)
                num_clipped: Any = counts
            else:
                if stats is not None:
                    num_clipped, rate = stats.num_clipped, stats.clipping_rate
                else:
                    num_clipped = float((aux.grad_norms > C).sum().item())
                    rate = aux.clipping_rate
                nxt = _update(C, rate, fold_in(state._rng_key, state._step))
            new_state = _next_state(state, nxt, num_clipped, float(batch_size))
            if return_aux:
                return (grads, AdaptiveClippedGradAux(
                    loss_values=aux.loss_values, grad_norms=aux.grad_norms,
                    clipped_grad_norms=aux.clipped_grad_norms, loss_aux=aux.loss_aux,
                    clipping_rate=aux.clipping_rate, batch_size=batch_size, group_norms=aux.group_norms,
                )), new_state
            if return_stats:
                return (grads, stats), new_state
            return grads, new_state

    grad_fn.engine = engine  # type: ignore[attr-defined]
    initial_state = AdaptiveClipState(
        _current_clipping_norm=initial_clipping_norm, _next_clipping_norm=initial_clipping_norm, _step=0,
        _rng_key=key, _fraction_noise_std=fraction_noise_std, _learning_rate=learning_rate,
        _target_quantile=target_quantile, _clipping_norm_min=clipping_norm_min,
        _clipping_norm_max=clipping_norm_max, _num_clipped=_empty_counts(), _batch_size=0,
    )
    return grad_fn, initial_state


__all__ = ["AdaptiveClipState", "AdaptiveClippedGradAux", "adaptive_clipped_grad"]
