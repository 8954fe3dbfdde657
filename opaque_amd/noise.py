"""``gaussian_noise``: drop-in for ``opaque.dpsgd.noise.gaussian_noise``.

Same factory signature, state, metadata and error behaviour as
``opaque-dpsgd/.../noise/_gaussian.py:147-407``.  The sampler runs on the
GPU (``odp_gaussian_noise``): one launch per call covers every leaf, and
element e of the flattened pytree (sorted-key order) draws its uniform from
a counter-based Philox4x32-10 stream keyed by the 64-bit seed of
``fold_in(key, step)`` (24 bits per element for float32 compute, the grid
of a float32 ``torch.rand``; 53 bits for float64), so noise at step t is a
pure function of (key, t) as in the reference.  The reference draws its
uniforms from a CPU mt19937 stream instead; both feed the same inverse-CDF
transform, clamps and bounded renormalisation.
"""

from __future__ import annotations

import dataclasses
import struct
from collections import OrderedDict

import numpy as np
import torch
from torch.autograd.profiler import record_function

from opaque_amd import _native as N
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


# Leaf dtypes of the noise kernel, and the compute dtypes it evaluates the
# inverse CDF in.
_LEAF_CODE = {torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16, torch.float16: N.DTYPE_F16,
              torch.float64: N.DTYPE_F64}
_COMPUTE_CODE = {torch.float32: N.DTYPE_F32, torch.float64: N.DTYPE_F64}


# Device copies of recent launch tables, keyed by their bytes: a training loop
# noises the same buffers with the same sigma every step, and a hit needs no
# host-to-device copy.  Tables hold addresses and sizes only, so a stale
# entry is never wrong, just unused.
_TABLES: OrderedDict[tuple, torch.Tensor] = OrderedDict()
_TABLES_MAX = 16


def _device_table(blob: np.ndarray, device: torch.device) -> torch.Tensor:
    k = (str(device), blob.tobytes())
    t = _TABLES.get(k)
    if t is not None:
        _TABLES.move_to_end(k)
        # Its memory is not reused before this stream's work that reads it.
        t.record_stream(torch.cuda.current_stream(device))
        return t
    # One pinned, asynchronous copy: the host does not wait for earlier work.
    host = torch.empty(blob.size, dtype=torch.uint8, pin_memory=True)
    host.numpy()[:] = blob
    t = host.to(device, non_blocking=True)
    _TABLES[k] = t
    if len(_TABLES) > _TABLES_MAX:
        _TABLES.popitem(last=False)
    return t


def add_noise_tree(pytree, stddev: float | PerGroup, seed: int, bound=None, tag: int = 0,
                   compute_dtype: torch.dtype = torch.float32):
    """Noise every tensor leaf of ``pytree`` with one device launch.

    Leaves with zero stddev (and no bound) are returned as the same tensor
    objects, as the reference's sampler returns its input.
    """
    _validate_stddev(stddev)
    if compute_dtype not in _COMPUTE_CODE:
        raise TypeError(f"compute_dtype must be torch.float32 or torch.float64, got {compute_dtype}")
    paths, leaves, td = tree_flatten_with_paths(pytree)
    out = list(leaves)
    rows, blocks = [], []
    lib = N.load()
    flat = 0
    device = None
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
        if t.dtype not in _LEAF_CODE:
            raise TypeError(f"gaussian_noise supports floating-point leaves, got {t.dtype} at {p!r}")
        src = t.detach().contiguous()
        dst = torch.empty_like(src)
        out[i] = dst.view(t.shape)
        if n == 0:
            continue
        code = _LEAF_CODE[src.dtype]
        rows.append([src.data_ptr(), dst.data_ptr(), n, off, _f64(sd), code | (code << 8), 0, 0])
        blocks.append(lib.odp_gaussian_noise_blocks(off, n))
    if rows:
        probs = np.asarray(rows, dtype=np.int64).reshape(-1)
        ws = np.zeros(len(blocks) + 1, dtype=np.int64)
        np.cumsum(blocks, out=ws[1:])
        total = int(ws[-1])
        if total >= 2**31 - 1:
            raise ValueError("gaussian_noise: the pytree exceeds one launch; noise it in parts")
        dev_tab = _device_table(np.concatenate([probs.view(np.uint8), ws.astype(np.int32).view(np.uint8)]),
                                device)
        stream = torch.cuda.current_stream(device).cuda_stream
        low, high = bound if bound is not None else (0.0, 0.0)
        N.check(
            lib.odp_gaussian_noise(stream, dev_tab.data_ptr(), dev_tab.data_ptr() + probs.size * 8, len(rows),
                                   total, seed & (2**64 - 1), tag, _COMPUTE_CODE[compute_dtype],
                                   1 if bound is not None else 0, float(low), float(high)),
            "odp_gaussian_noise",
        )
        # The sources return to torch's caching allocator, which orders their
        # reuse after this launch.
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
    if compute_dtype not in _COMPUTE_CODE:
        raise TypeError(
            "opaque_amd.gaussian_noise evaluates the inverse CDF in float32 or float64 on the device; "
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
        n1 = add_noise_tree(first.pytree, s1, k1.seed, rbound, compute_dtype=compute_dtype)
        n2 = add_noise_tree(second.pytree, s2, k2.seed, rbound, compute_dtype=compute_dtype)
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
            noisy = add_noise_tree(grads.pytree, sd, step_key.seed, rbound, compute_dtype=compute_dtype)
            return NoisedPytree(pytree=noisy, max_norm=grads.max_norm, noise_stddev=sd), nxt

    return noise_fn, state


__all__ = ["GaussianNoiseState", "add_noise_tree", "gaussian_noise"]
