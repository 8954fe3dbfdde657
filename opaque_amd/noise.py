"""``gaussian_noise``: drop-in for ``opaque.dpsgd.noise.gaussian_noise``.

Same factory signature, state, metadata and error behaviour as
``opaque-dpsgd/.../noise/_gaussian.py:147-407``.  The sampler runs on the
GPU (``odp_gaussian_noise``): one launch per call covers every leaf, and
element e of the flattened pytree (sorted-key order) draws from the
Philox4x32-10 block e >> 2 keyed by the 64-bit seed of
``fold_in(key, step)``, so noise at step t is a pure function of (key, t)
as in the reference.  The reference draws its uniforms from a CPU mt19937
stream instead; both feed the same inverse-CDF transform.
"""

from __future__ import annotations

import dataclasses
import struct

import numpy as np
import torch
from torch.autograd.profiler import record_function

from opaque_amd import _native as N
from opaque_amd.engine import dtype_code
from opaque_amd.noise_allocation import (
    PAIRED_FIRST_STREAM_FOLD,
    PAIRED_SECOND_STREAM_FOLD,
    per_group_noise_stddev,
    resolve_paired_clipped,
)
from opaque_amd.pytree import tree_flatten_with_paths, tree_unflatten
from opaque_amd.random import RngKey, fold_in
from opaque_amd.types import (
    ClippedPytree,
    NoisedPytree,
    NoiseState,
    PerGroup,
    SecondMomentClippingOutput,
    SecondMomentNoiseOutput,
)


@dataclasses.dataclass(frozen=True)
class GaussianNoiseState(NoiseState):
    """Noise for step t is derived from fold_in(_rng_key, t)."""

    _step_counter: int
    _rng_key: RngKey


def _validate_stddev(sd: float | PerGroup) -> None:
    if isinstance(sd, PerGroup):
        for name, v in sd.values.items():
            if v < 0:
                raise ValueError(
                    "noise standard deviation must be non-negative for all groups, "
                    f"got {v} for group '{name}'"
                )
    elif sd < 0:
        raise ValueError(f"noise standard deviation must be non-negative, got {sd}")


def _resolve_bound(bound) -> tuple[float, float] | None:
    if bound is None:
        return None
    if isinstance(bound, (tuple, list)):
        if len(bound) != 2:
            raise ValueError(
                f"bound must be a 2-tuple (low, high) when given a sequence, got length {len(bound)}"
            )
        low, high = float(bound[0]), float(bound[1])
    else:
        b = float(bound)
        if b <= 0:
            raise ValueError(f"scalar bound must be positive (interpreted as [-B, B]), got {b}")
        low, high = -b, b
    if not low < high:
        raise ValueError(f"bound must satisfy low < high, got ({low}, {high})")
    if not low <= 0.0 <= high:
        raise ValueError(
            "bound must straddle zero (low <= 0 <= high) so the support "
            f"contains the unbiased mechanism centre, got ({low}, {high})"
        )
    return low, high


def _f64(x: float) -> int:
    return struct.unpack("<q", struct.pack("<d", float(x)))[0]


def add_noise_tree(pytree, stddev: float | PerGroup, seed: int, bound=None, tag: int = 0):
    """Noise every tensor leaf of ``pytree`` with one device launch.

    Leaves with zero stddev (and no bound) are returned as the same tensor
    objects, as the reference's sampler returns its input.
    """
    _validate_stddev(stddev)
    paths, leaves, td = tree_flatten_with_paths(pytree)
    out = list(leaves)
    rows, blocks = [], []
    lib = N.load()
    flat = 0
    device = None
    keep = []
    for i, (p, t) in enumerate(zip(paths, leaves)):
        if not isinstance(t, torch.Tensor):
            if isinstance(stddev, PerGroup):
                raise TypeError(
                    "gaussian_noise with PerGroup stddev expects tensor "
                    f"leaves; got {type(t).__name__} at path {p!r}."
                )
            continue
        sd = float(stddev.for_path(p)) if isinstance(stddev, PerGroup) else float(stddev)
        n = t.numel()
        off = flat
        flat += n
        if sd == 0.0 and bound is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "opaque_amd.gaussian_noise runs on the GPU; got a leaf on "
                f"{t.device} at path {p!r}. Move the clipped gradients to the device first."
            )
        if device is None:
            device = t.device
        if t.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"gaussian_noise supports float32/bfloat16 leaves, got {t.dtype} at {p!r}")
        src = t.detach().contiguous()
        keep.append(src)
        dst = torch.empty_like(src)
        out[i] = dst.view(t.shape)
        if n == 0:
            continue
        low, high = bound if bound is not None else (0.0, 0.0)
        dts = dtype_code(src.dtype) | (dtype_code(dst.dtype) << 8) | ((1 if bound is not None else 0) << 16)
        rows.append([src.data_ptr(), dst.data_ptr(), n, off, _f64(sd), dts, _f64(low), _f64(high)])
        blocks.append(lib.odp_gaussian_noise_blocks(off, n))
    if rows:
        probs = torch.tensor(np.asarray(rows, dtype=np.int64), device=device)
        ws = np.zeros(len(blocks) + 1, dtype=np.int64)
        np.cumsum(blocks, out=ws[1:])
        total = int(ws[-1])
        ws_d = torch.tensor(ws.astype(np.int32), device=device)
        stream = torch.cuda.current_stream(device).cuda_stream
        N.check(
            lib.odp_gaussian_noise(stream, probs.data_ptr(), ws_d.data_ptr(), len(rows), total,
                                   seed & (2**64 - 1), tag),
            "odp_gaussian_noise",
        )
        # `keep`, probs and ws_d return to the caching allocator, whose reuse is
        # ordered after this launch on the same stream.
    return tree_unflatten(td, out)


def gaussian_noise(
    *,
    noise_multiplier: float,
    key: RngKey,
    bound: float | tuple[float, float] | list[float] | None = None,
    compute_dtype: torch.dtype = torch.float32,
):
    """Create ``(noise_fn, GaussianNoiseState)``; see the module docstring."""
    if noise_multiplier is None:
        raise ValueError("gaussian_noise() requires noise_multiplier.")
    nm = float(noise_multiplier)
    if nm < 0:
        raise ValueError(f"noise_multiplier must be non-negative, got {noise_multiplier}")
    rbound = _resolve_bound(bound)
    if not isinstance(key, RngKey):
        raise TypeError(f"key must be RngKey, got {type(key)}")
    if compute_dtype != torch.float32:
        raise TypeError(
            "opaque_amd.gaussian_noise evaluates the inverse CDF in float32 on the device; "
            f"compute_dtype={compute_dtype} is not supported"
        )
    state = GaussianNoiseState(_step_counter=0, _rng_key=key)

    def _stddev(c: ClippedPytree) -> float | PerGroup:
        if isinstance(c.max_norm, PerGroup):
            return per_group_noise_stddev(c.max_norm, nm)
        eff = 0.0 if nm == 0.0 else nm * c.max_norm
        _validate_stddev(eff)
        return eff

    def _paired(x: SecondMomentClippingOutput, st: GaussianNoiseState):
        first, second, s1, s2 = resolve_paired_clipped(x, noise_multiplier=nm)
        k1 = fold_in(fold_in(st._rng_key, PAIRED_FIRST_STREAM_FOLD), st._step_counter)
        k2 = fold_in(fold_in(st._rng_key, PAIRED_SECOND_STREAM_FOLD), st._step_counter)
        n1 = add_noise_tree(first.pytree, s1, k1.seed, rbound)
        n2 = add_noise_tree(second.pytree, s2, k2.seed, rbound)
        nxt = GaussianNoiseState(_step_counter=st._step_counter + 1, _rng_key=st._rng_key)
        return (
            SecondMomentNoiseOutput(
                NoisedPytree(pytree=n1, max_norm=first.max_norm, noise_stddev=s1),
                NoisedPytree(pytree=n2, max_norm=second.max_norm, noise_stddev=s2),
            ),
            nxt,
        )

    def noise_fn(grads, st):
        with record_function("opaque::gaussian_noise"):
            if isinstance(grads, SecondMomentClippingOutput):
                return _paired(grads, st)
            nxt = GaussianNoiseState(_step_counter=st._step_counter + 1, _rng_key=st._rng_key)
            if isinstance(grads, NoisedPytree):
                raise TypeError(
                    "gaussian_noise expects ClippedPytree inputs, not NoisedPytree "
                    "values that have already passed through a noise mechanism."
                )
            if not isinstance(grads, ClippedPytree):
                raise TypeError(
                    "gaussian_noise expects ClippedPytree inputs. Wrap manual "
                    "values with opaque.types.clipped(...)."
                )
            sd = _stddev(grads)
            step_key = fold_in(st._rng_key, st._step_counter)
            noisy = add_noise_tree(grads.pytree, sd, step_key.seed, rbound)
            return NoisedPytree(pytree=noisy, max_norm=grads.max_norm, noise_stddev=sd), nxt

    return noise_fn, state


__all__ = ["GaussianNoiseState", "add_noise_tree", "gaussian_noise"]
