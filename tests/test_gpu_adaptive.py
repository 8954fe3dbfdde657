"""GPU runs of ``adaptive_clipped_grad`` (the threshold update around the native clip kernels)."""

from __future__ import annotations

import math

import pytest
import torch

from opaque_amd.adaptive import AdaptiveClipState, AdaptiveClippedGradAux, adaptive_clipped_grad
from opaque_amd.clipping import ClippingStats, per_group
from opaque_amd.random import fold_in, generator_from_key, key
from opaque_amd.types import ClippedPytree, PerGroup

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _loss(params, x):
    return (params * x).sum()


@pytest.mark.parametrize("target_quantile", [0.3, 0.7])
def test_threshold_converges_to_target_quantile(target_quantile):
    # Reference test_adaptive.py:360-387: per-example norms 0.1 .. 10.
    norms = torch.arange(1, 101, dtype=torch.float32) / 10.0
    batch_x = torch.zeros(100, 4)
    batch_x[:, 0] = norms
    params = torch.zeros(4, device=DEV)
    grad_fn, st = adaptive_clipped_grad(_loss, initial_clipping_norm=1.0, target_quantile=target_quantile,
                                        learning_rate=0.5, fraction_noise_std=1e-6, key=key(0),
                                        batch_argnums=(1,))
    bx = batch_x.to(DEV)
    for _ in range(200):
        _, st = grad_fn(params, bx, state=st)
    frac = float((norms > st._current_clipping_norm).float().mean())
    assert frac == pytest.approx(target_quantile, abs=0.02)


def test_one_step_matches_the_update_rule():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, 6, generator=g) * torch.logspace(-1, 1, 16).view(16, 1)
    params = torch.zeros(6, device=DEV)
    grad_fn, st = adaptive_clipped_grad(_loss, initial_clipping_norm=2.0, key=key(9), return_aux=True,
                                        batch_argnums=(1,), normalize_by=16.0)
    (grads, aux), st1 = grad_fn(params, x.to(DEV), state=st)
    assert isinstance(grads, ClippedPytree) and grads.max_norm == 2.0 / 16.0
    assert isinstance(aux, AdaptiveClippedGradAux) and isinstance(st1, AdaptiveClipState)
    norms = x.norm(dim=1)
    rate = float((norms > 2.0).float().mean())
    noise = torch.randn(1, generator=generator_from_key(fold_in(key(9), 0))).item() * 0.05
    want = 2.0 * torch.exp(torch.tensor(0.2 * (rate + noise - 0.5))).item()
    assert st1._next_clipping_norm == pytest.approx(want, rel=1e-6)
    assert st1._current_clipping_norm == 2.0 and st1._step == 1 and st1._batch_size == 16.0
    assert aux.clipping_rate == pytest.approx(rate)
    # The clipped sum itself: per-example gradients are the rows of x.
    scale = torch.clamp(2.0 / norms, max=1.0)
    want_g = (scale[:, None] * x).sum(0) / 16.0
    assert torch.allclose(grads.pytree.cpu(), want_g, rtol=1e-5, atol=1e-6)


def test_per_group_thresholds_and_stats():
    params = {"a": torch.zeros(3, device=DEV), "b": torch.zeros(2, device=DEV)}
    pg = per_group(params, a=1.0, b=0.5)

    def loss(p, x):
        return (p["a"] * x[:3]).sum() + (p["b"] * x[3:]).sum()

    g = torch.Generator().manual_seed(4)
    x = torch.randn(12, 5, generator=g).to(DEV)
    grad_fn, st = adaptive_clipped_grad(loss, initial_clipping_norm=pg, key=key(1), return_stats=True)
    (grads, stats), st1 = grad_fn(params, x, state=st)
    assert isinstance(stats, ClippingStats) and isinstance(stats.num_clipped, dict)
    assert isinstance(st1._next_clipping_norm, PerGroup)
    for i, name in enumerate(sorted(pg.values)):
        rate = stats.clipping_rate[name]
        noise = torch.randn(1, generator=generator_from_key(fold_in(fold_in(key(1), 0), i))).item() * 0.05
        want = pg.values[name] * math.exp(0.2 * (rate + noise - 0.5))
        assert st1._next_clipping_norm.values[name] == pytest.approx(want, rel=1e-6)
