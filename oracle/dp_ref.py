"""CPU restatement of the reference clip / sum / noise algorithm (test oracle).

Every function names the reference lines it restates (paths relative to the
reference's packages/; ENG = opaque-engine/src/opaque/api/engine,
DPS = opaque-dpsgd/src/opaque/api/dpsgd).  Pure torch on the CPU.
"""

from __future__ import annotations

import hashlib
import math
from typing import Any, Callable

import torch

# ---------------------------------------------------------------------------
# Pytree order: dict keys sorted, sequences by index (ENG/pytree.py:67-77,150-152)
# ---------------------------------------------------------------------------


def flatten(tree: Any, path: tuple = ()) -> list[tuple[tuple, Any]]:
    if tree is None:
        return []
    if isinstance(tree, dict):
        out = []
        for k in sorted(tree):
            out.extend(flatten(tree[k], path + (k,)))
        return out
    if isinstance(tree, (list, tuple)):
        out = []
        for i, v in enumerate(tree):
            out.extend(flatten(v, path + (i,)))
        return out
    return [(path, tree)]


def rebuild(tree: Any, values: dict[tuple, Any], path: tuple = ()) -> Any:
    if tree is None:
        return None
    if isinstance(tree, dict):
        return {k: rebuild(v, values, path + (k,)) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        vals = [rebuild(v, values, path + (i,)) for i, v in enumerate(tree)]
        return type(tree)(vals) if not hasattr(type(tree), "_fields") else type(tree)(*vals)
    return values[path]


def global_norm(tree: Any) -> torch.Tensor:
    """sqrt(sum ||leaf||^2) in at-least-float32 (ENG/pytree.py:336-430)."""
    leaves = [x for _, x in flatten(tree) if isinstance(x, torch.Tensor)]
    acc = torch.float32
    for t in leaves:
        if t.is_floating_point():
            acc = torch.promote_types(acc, t.dtype)
    total = torch.zeros((), dtype=acc)
    for t in leaves:
        x = t.to(acc)
        total = total + (x * x).sum(dtype=acc)
    return torch.sqrt(total)


# ---------------------------------------------------------------------------
# RNG keys (ENG/random/_engine.py:27-101)
# ---------------------------------------------------------------------------


def _blake64(*parts: object) -> int:
    h = hashlib.blake2b(digest_size=8)
    for p in parts:
        h.update(p.to_bytes(16, "little", signed=True) if isinstance(p, int) else str(p).encode())
        h.update(b"|")
    return int.from_bytes(h.digest(), "little")


def key_seed(seed: int) -> int:
    return seed & (2**64 - 1)


def fold_in_seed(seed: int, *data: int | str) -> int:
    for d in data:
        seed = _blake64(seed, d)
    return seed


# ---------------------------------------------------------------------------
# Guard constants (ENG/clipping/_pytree.py:81-142,156-221)
# ---------------------------------------------------------------------------

_BLOCK = 2048
_BLOCKED_MIN = 4096


def acc_dtype(leaves: list[torch.Tensor], compute_dtype: torch.dtype | None) -> torch.dtype:
    if compute_dtype is not None:
        return compute_dtype
    acc = torch.float32
    for t in leaves:
        if t.is_floating_point():
            acc = torch.promote_types(acc, torch.float32 if t.dtype in (torch.float16, torch.bfloat16) else t.dtype)
    return acc


def reduction_terms(leaves: list[torch.Tensor]) -> int:
    widest = max((t.numel() for t in leaves), default=0)
    if widest <= 1:
        return 0
    if widest > _BLOCKED_MIN:
        return _BLOCK + (widest + _BLOCK - 1) // _BLOCK
    return widest


def roundoff(acc: torch.dtype, n_leaves: int, n_red: int) -> float:
    u_acc = torch.finfo(acc).eps / 2.0
    u_sq = torch.finfo(torch.float64).eps / 2.0
    return (u_acc + (max(n_leaves, 1) + n_red) * u_sq) / 2.0


def finalize(ratio: torch.Tensor, store: torch.dtype, rnd: float, clamp_one: bool) -> torch.Tensor:
    """Guarded scale: ratio*rel - abs, [min 1], non-finite -> 0, >= 0."""
    if store.is_floating_point:
        fi = torch.finfo(store)
        rel = 1.0 - 2.0 * (fi.eps / 2.0 + rnd)
        scale = ratio * rel - fi.smallest_normal * fi.eps
    else:
        scale = ratio
    if clamp_one:
        scale = torch.minimum(torch.ones_like(scale), scale)
    scale = torch.where(torch.isfinite(scale), scale, torch.zeros_like(scale))
    return torch.clamp(scale, min=0.0)


def leaf_sq_sum(t: torch.Tensor, acc: torch.dtype) -> torch.Tensor:
    """Squares in `acc`, two-stage fp64 sum above 4096 elements (_pytree.py:224-252)."""
    x = t.to(acc)
    flat = (x * x).reshape(-1)
    n = flat.numel()
    if n <= _BLOCKED_MIN:
        return flat.sum(dtype=torch.float64)
    main = n // _BLOCK * _BLOCK
    total = flat[:main].reshape(-1, _BLOCK).sum(-1, dtype=torch.float64).sum(dtype=torch.float64)
    if main < n:
        total = total + flat[main:].sum(dtype=torch.float64)
    return total


# ---------------------------------------------------------------------------
# Per-example scaling (ENG/clipping/_pytree.py:345-564)
# ---------------------------------------------------------------------------


def _scale_tree(tree, C, *, autos: bool, gamma: float, compute_dtype, return_zero=False):
    items = flatten(tree)
    items = [(p, torch.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0)) for p, x in items]
    leaves = [x for _, x in items]
    acc = acc_dtype(leaves, compute_dtype)
    rnd = roundoff(acc, len(leaves), reduction_terms(leaves))
    sq = {p: leaf_sq_sum(x, acc) for p, x in items}
    total = torch.zeros((), dtype=torch.float64)
    for p, _ in items:
        total = total + sq[p]
    norm = torch.sqrt(total)

    def ratio_for(n: torch.Tensor, c: float) -> torch.Tensor:
        c_t = torch.clamp(torch.tensor(c, dtype=torch.float64), min=0.0)
        return c_t / (n + torch.tensor(gamma, dtype=torch.float64)) if autos else c_t / n

    group_norms = None
    if hasattr(C, "groups"):
        paths = {p for p, _ in items}
        if paths != set(C.groups):
            raise ValueError("PerGroup path keys must match the pytree tensor leaves exactly.")
        gsq: dict[str, torch.Tensor] = {}
        for p, _ in items:
            g = C.groups[p]
            gsq[g] = sq[p] if g not in gsq else gsq[g] + sq[p]
        gn = {g: torch.sqrt(v) for g, v in gsq.items()}
        ratios = {g: ratio_for(gn[g], C.values[g]) for g in gn}
        scaled = {p: finalize(ratios[C.groups[p]], x.dtype, rnd, not autos).to(x.dtype) * x for p, x in items}
        group_norms = {g: v.to(acc) for g, v in gn.items()}
    else:
        ratio = ratio_for(norm, C)
        scaled = {p: finalize(ratio, x.dtype, rnd, not autos).to(x.dtype) * x for p, x in items}
    if return_zero:
        scaled = {p: torch.zeros_like(v) for p, v in scaled.items()}
    return rebuild(tree, scaled), norm.to(acc), group_norms


def clip_pytree(tree, clipping_norm, return_zero=False, *, compute_dtype=None):
    """clip_pytree (ENG/clipping/_pytree.py:475-564); returns (clipped, norm, group_norms)."""
    return _scale_tree(tree, clipping_norm, autos=False, gamma=0.0, compute_dtype=compute_dtype,
                       return_zero=return_zero)


def auto_scale_pytree(tree, R=1.0, gamma=0.01, *, compute_dtype=None):
    """auto_scale_pytree (ENG/clipping/_pytree.py:345-431)."""
    if gamma <= 0:
        raise ValueError(f"gamma must be positive, got {gamma}")
    return _scale_tree(tree, R, autos=True, gamma=gamma, compute_dtype=compute_dtype)


# ---------------------------------------------------------------------------
# clipped_grad (ENG/clipping/_clipped_grad.py:81-341, _clipped_fun.py:526-881)
# ---------------------------------------------------------------------------


def _sum_dtype(x: torch.Tensor, compute_dtype):
    if compute_dtype is not None:
        return compute_dtype
    return torch.float32 if x.dtype in (torch.float16, torch.bfloat16) else None


def clipped_grad(
    loss_fn: Callable,
    params: Any,
    batch: tuple,
    *,
    clipping_norm: Any = 1.0,
    normalize_by: float = 1.0,
    autos: bool = False,
    gamma: float = 0.01,
    dtype: torch.dtype | None = None,
    compute_dtype: torch.dtype | None = None,
    second_moment: bool = False,
):
    """vmap(grad_and_value) per example, scale, fp32-accumulated sum, /normalize_by.

    ``loss_fn(params, *batch_i)`` is the per-example loss.  Returns
    ``(summed_tree, aux)`` with aux keys ``norms``, ``group_norms``,
    ``loss_values``, ``clipped_norms``, ``per_example`` and ``squared``.
    """
    gv = torch.func.grad_and_value(loss_fn, argnums=0)

    def per_example(p, *b):
        g, v = gv(p, *b)
        return g, v

    in_dims = (None,) + (0,) * len(batch)
    grads, values = torch.func.vmap(per_example, in_dims=in_dims, randomness="same")(params, *batch)
    n = values.shape[0]
    items = flatten(grads)
    outs = {p: [] for p, _ in items}
    norms, cnorms, gnorms = [], [], []
    for i in range(n):
        ex = rebuild(grads, {p: x[i] for p, x in items})
        if autos:
            scaled, nrm, gn = auto_scale_pytree(ex, clipping_norm, gamma, compute_dtype=compute_dtype)
        else:
            scaled, nrm, gn = clip_pytree(ex, clipping_norm, compute_dtype=compute_dtype)
        norms.append(nrm)
        gnorms.append(gn)
        cnorms.append(global_norm(scaled))
        for p, x in flatten(scaled):
            outs[p].append(x)
    summed, squared, stacked = {}, {}, {}
    for p, _ in items:
        st = torch.stack(outs[p])
        stacked[p] = st
        acc = _sum_dtype(st, compute_dtype)
        target = dtype if dtype is not None else st.dtype
        s = torch.sum(st, dim=0, dtype=acc)
        s = s.to(target) if s.dtype != target else s
        if normalize_by != 1.0:
            s = s / normalize_by
        summed[p] = s
        if second_moment:
            sq = st.square()
            s2 = torch.sum(sq, dim=0, dtype=acc)
            s2 = s2.to(target) if s2.dtype != target else s2
            if normalize_by != 1.0:
                s2 = s2 / normalize_by
            squared[p] = s2
    aux = {
        "norms": torch.stack(norms),
        "group_norms": None if gnorms[0] is None else {g: torch.stack([d[g] for d in gnorms]) for g in gnorms[0]},
        "loss_values": values.detach(),
        "clipped_norms": torch.stack(cnorms),
        "per_example": rebuild(grads, stacked),
        "squared": rebuild(grads, squared) if second_moment else None,
    }
    return rebuild(grads, summed), aux


def clipped_count(norms: torch.Tensor, threshold: float) -> int:
    """num_clipped = #(norm > C) in the norms' dtype (_clipped_fun.py:512-523)."""
    return int((norms > threshold).sum().item())


# ---------------------------------------------------------------------------
# Gaussian noise with the reference's CPU stream (DPS/noise/_gaussian.py:235-301,370-405)
# ---------------------------------------------------------------------------


def gaussian_noise_reference(tree, stddev, key: int, step: int, compute_dtype=torch.float32, bound=None,
                             stream_fold: int | None = None):
    """The reference's CPU sampler (DPS/noise/_gaussian.py:235-301,317-405).

    A CPU ``torch.Generator`` seeded by ``fold_in(key, step)`` (or
    ``fold_in(fold_in(key, stream_fold), step)`` for the paired streams,
    :329-334) reduced modulo 2^63 - 1 (ENG/random/_engine.py:98-101) draws
    ``torch.rand`` uniforms leaf by leaf in sorted-key order; a leaf whose
    stddev is 0 draws nothing and is returned (clamped to the bound, if any).
    ``stddev`` is a float or a dict path -> float (per-group sigma).
    """
    seed = fold_in_seed(key_seed(key), step) if stream_fold is None else \
        fold_in_seed(key_seed(key), stream_fold, step)
    gen = torch.Generator().manual_seed(seed % (2**63 - 1))
    eps = torch.finfo(compute_dtype).eps
    sqrt2 = math.sqrt(2.0)
    out = {}
    for p, c in flatten(tree):
        sd = float(stddev[p]) if isinstance(stddev, dict) else float(stddev)
        if sd == 0:
            out[p] = c if bound is None else torch.clamp(c, min=bound[0], max=bound[1])
            continue
        u = torch.rand(c.shape, dtype=compute_dtype, generator=gen)
        cc = c.to(compute_dtype) if c.dtype != compute_dtype else c
        if bound is None:
            u = torch.clamp(u, min=eps, max=1.0 - eps)
            x = cc + sd * sqrt2 * torch.erfinv(2.0 * u - 1.0)
        else:
            low, high = bound
            z_low, z_high = (low - cc) / sd, (high - cc) / sd
            alpha = 0.5 * (1.0 + torch.erf(z_low / sqrt2))
            beta = 0.5 * (1.0 + torch.erf(z_high / sqrt2))
            u = torch.clamp(alpha + u * (beta - alpha), min=eps, max=1.0 - eps)
            x = torch.clamp(cc + sd * sqrt2 * torch.erfinv(2.0 * u - 1.0), min=low, max=high)
        out[p] = x.to(c.dtype) if c.dtype != compute_dtype else x
    return rebuild(tree, out)


def per_group_sigma(values: dict[str, float], nm: float) -> dict[str, float]:
    """sigma_g = nm * sqrt(C_g * sum C) (ENG/noise_allocation.py:33-95)."""
    if nm == 0.0:
        return dict.fromkeys(values, 0.0)
    tot = sum(values.values())
    return {k: nm * math.sqrt(c * tot) for k, c in values.items()}
