"""Per-example clipping: drop-in ``clipped_grad`` / ``auto_clipped_grad`` / ``per_group``.

Same factories, call convention, states, aux types, validation and error
messages as the reference (``opaque-engine/.../clipping/_clipped_grad.py:31-341``,
``_clipped_fun.py:26-74,194-205,472-523``, ``_auto.py:30-354``,
``_per_group.py:41-152``).  The arithmetic runs in the native kernels of
``libopaque_dp.so`` on the current HIP stream; there is no CPU route.

Two ways to obtain the per-example gradients feed the same kernels:

* **Seam capture.**  When the loss function applies its LoRA adapters
  through :mod:`opaque_amd.capture` (``lora_linear``, ``peft_lora_linear``,
  ``LoRALinear``), a one-example discovery pass finds the adapter factors
  that reach the loss only through a seam.  One batched forward/backward
  then records the activations ``x`` and output gradients ``g`` of every
  seam, and ``GhostPlan`` turns them into per-example factor gradients,
  norms, clip scales and the clipped sum without autograd ever
  materialising a per-example gradient.  Every other trainable leaf gets
  its per-example gradient from the same backward pass through a
  batch-expanded copy of the leaf.
* **Materialised.**  Otherwise (no seams, a ``pre_clipping_transform``,
  a ``_scale_fn``) ``torch.func.vmap(grad_and_value)`` produces the
  per-example gradients on the device, as the reference does, and the
  kernels compute norms, scales and the sum.
"""

from __future__ import annotations

from collections.abc import Callable
from dataclasses import dataclass
import time
from typing import Any

import torch
from torch.autograd.profiler import record_function

from opaque_amd import _native as N
from opaque_amd.capture import CaptureSession, SiteRecord
from opaque_amd.engine import (
    LORA_PTRS,
    ClipSpec,
    GhostPlan,
    LeafOut,
    LinearSite,
    LoraSite,
    MaterializedLeaf,
    Segments,
    leaves_key,
    plan_key,
    supports_rows,
)
from opaque_amd.guard import guard_constants, leaf_guards
from opaque_amd.pytree import (
    param_path_display,
    tree_flatten_with_paths,
    tree_map,
    tree_unflatten,
)
from opaque_amd.types import (
    ClippedPytree,
    ClipState,
    PerGroup,
    SecondMomentClippingOutput,
    clipped,
)

_KERNEL_DTYPES = (torch.float32, torch.bfloat16)  # the seam-capture kernels
_LEAF_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float64)  # materialised leaves
_DEFAULT_GAMMA = 0.01


def _identity(x: Any) -> Any:
    return x


# ---------------------------------------------------------------------------
# States and aux types (_clipped_fun.py:26-74, _clipped_grad.py:31-58, _auto.py:47-83)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class FixedClipState(ClipState):
    """Marker state of fixed-threshold clipping (the threshold travels in ``max_norm``)."""


@dataclass(frozen=True)
class AutoClipState(ClipState):
    """Marker state of AUTO-S scaling."""


@dataclass(frozen=True)
class ClippedGradAux:
    """Per-example diagnostics: pre-noise values, not for private computation."""

    loss_values: Any | None = None
    grad_norms: Any | None = None
    clipped_grad_norms: Any | None = None
    loss_aux: Any | None = None
    clipping_rate: float | None = None
    batch_size: int = 0
    group_norms: dict[str, torch.Tensor] | None = None


@dataclass(frozen=True)
class AutoClippedGradAux(ClippedGradAux):
    """``ClippedGradAux`` with AUTO-S semantics for the norms."""


@dataclass(frozen=True)
class ClippingStats:
    """Aggregated clipping statistics without per-example outputs."""

    num_clipped: float | dict[str, float]
    clipping_rate: float | dict[str, float] | None
    batch_size: int = 0
    all_finite: bool = True


# ---------------------------------------------------------------------------
# Validation (_clipped_grad.py:61-78, _clipped_fun.py:194-205, _auto.py:94-105)
# ---------------------------------------------------------------------------


def _to_tuple(value: int | tuple[int, ...]) -> tuple[int, ...]:
    return (value,) if isinstance(value, int) else tuple(value)


def _validate_static_args(argnums, batch_argnums, normalize_by) -> None:
    if normalize_by <= 0.0:
        raise ValueError(f"normalize_by must be > 0, got {normalize_by}.")
    argnums = _to_tuple(argnums)
    batch_argnums = _to_tuple(batch_argnums)
    if not batch_argnums:
        raise ValueError("Batch argnums must not be empty.")
    if min(argnums + batch_argnums) < 0:
        raise ValueError(f"argnums={argnums} and batch_argnums={batch_argnums} must be >= 0.")
    shared = set(argnums) & set(batch_argnums)
    if shared:
        raise ValueError(
            "Cannot compute clipped gradients for argnums that have a batch axis. "
            f"argnums={argnums!r} and batch_argnums={batch_argnums!r} with overlap {list(shared)}."
        )


def _validate_clipping_norm(clipping_norm: float | PerGroup) -> None:
    if isinstance(clipping_norm, PerGroup):
        for name, value in clipping_norm.values.items():
            if value <= 0:
                raise ValueError(
                    f"clipping_norm must be positive for all groups, got {value} for group '{name}'"
                )
        return
    if clipping_norm <= 0:
        raise ValueError(f"clipping_norm must be positive, got {clipping_norm}")


def _validate_auto_params(R: float | PerGroup, gamma: float) -> None:
    if isinstance(R, PerGroup):
        for name, value in R.values.items():
            if value <= 0:
                raise ValueError(f"R must be positive for all groups, got {value} for group '{name}'")
    elif R <= 0:
        raise ValueError(f"R must be positive, got {R}")
    if gamma <= 0:
        raise ValueError(f"gamma must be positive, got {gamma}")


def _validate_per_group_paths(paths: list, pg: PerGroup) -> None:
    leaf_set, group_set = set(paths), set(pg.groups)
    if leaf_set == group_set:
        return
    parts = ["PerGroup path keys must match the pytree tensor leaves exactly."]
    missing_in_groups = sorted(leaf_set - group_set, key=param_path_display)
    missing_in_tree = sorted(group_set - leaf_set, key=param_path_display)
    if missing_in_groups:
        parts.append(f"Leaves with no group assignment: {missing_in_groups}.")
    if missing_in_tree:
        parts.append(f"Group paths with no matching leaf: {missing_in_tree}.")
    raise ValueError(" ".join(parts))


def batch_size_from_args(args: tuple, batch_argnums: tuple[int, ...]) -> int:
    """Batch size from the first tensor of the first batch argument (_helpers.py:38-73)."""
    first = args[batch_argnums[0]]
    if isinstance(first, torch.Tensor):
        return first.shape[0]
    tensors = [x for x in tree_flatten_with_paths(first)[1] if isinstance(x, torch.Tensor)]
    if not tensors:
        raise ValueError(
            f"Could not determine batch size: no tensor in batch arg at index {batch_argnums[0]}"
        )
    if tensors[0].ndim < 1:
        raise ValueError(
            "Expected batch tensor with ndim >= 1, got 0-d tensor in batch arg at index "
            f"{batch_argnums[0]}"
        )
    return tensors[0].shape[0]


def _zero_grads_like(args: tuple, argnums: tuple[int, ...]) -> Any:
    zeros = tuple(tree_map(torch.zeros_like, args[i]) for i in argnums)
    return zeros[0] if len(zeros) == 1 else zeros


# ---------------------------------------------------------------------------
# per_group (_per_group.py:41-152)
# ---------------------------------------------------------------------------


def per_group(
    params: Any,
    /,
    patterns: dict[str, float] | None = None,
    *,
    fallback: float | None = None,
    **kwargs: float,
) -> PerGroup:
    """PerGroup from substring patterns over the leaves' dotted paths (exactly one match each)."""
    all_patterns: dict[str, float] = {}
    if patterns is not None:
        all_patterns.update(patterns)
    all_patterns.update(kwargs)
    if not all_patterns and fallback is None:
        raise ValueError("At least one pattern must be provided.")
    for pat, val in all_patterns.items():
        if val <= 0:
            raise ValueError(f"Per-group value must be positive, got {val} for pattern '{pat}'.")
    if fallback is not None and fallback <= 0:
        raise ValueError(f"Fallback value must be positive, got {fallback}.")
    paths, leaves, _ = tree_flatten_with_paths(params)
    groups: dict = {}
    for path, leaf in zip(paths, leaves):
        if not isinstance(leaf, torch.Tensor):
            raise TypeError(
                f"Expected tensor leaves for per-group clipping; got {type(leaf).__name__} at path {path!r}."
            )
        display = param_path_display(path)
        matches = [pat for pat in all_patterns if pat in display]
        if not matches:
            if fallback is not None:
                groups[path] = "fallback"
                continue
            raise ValueError(
                f"Parameter path {path!r} (display {display!r}) did not match any pattern. "
                f"Available patterns: {list(all_patterns.keys())}. "
                "Use fallback=<value> to catch unmatched parameters."
            )
        if len(matches) > 1:
            raise ValueError(
                f"Parameter path {path!r} (display {display!r}) matched multiple patterns: {matches}. "
                "Each parameter must match exactly one pattern."
            )
        groups[path] = matches[0]
    used = set(groups.values())
    values = {pat: float(v) for pat, v in all_patterns.items() if pat in used}
    if fallback is not None and "fallback" in used:
        values["fallback"] = float(fallback)
    return PerGroup(groups=groups, values=values)


# ---------------------------------------------------------------------------
# The engine behind a clipped_grad factory
# ---------------------------------------------------------------------------


@dataclass
class _StepOut:
    """What one (micro)batch produced on the device."""

    leaves: list[torch.Tensor]
    squared: list[torch.Tensor] | None
    norms: torch.Tensor
    group_norms: torch.Tensor  # [G, n]
    clipped: torch.Tensor  # [G, n] uint8
    clipped_total: torch.Tensor  # [n] uint8
    clipped_norms: torch.Tensor
    values: torch.Tensor | None
    loss_aux: Any
    all_finite: torch.Tensor | None


class _Discovery:
    """Which gradient leaves reach the loss through exactly one LoRA seam and nowhere else."""

    def __init__(self, eligible: frozenset[int]) -> None:
        self.eligible = eligible


class _ClipEngine:
    def __init__(
        self,
        loss_fn: Callable,
        argnums: tuple[int, ...],
        argnums_raw: int | tuple[int, ...],
        has_aux: bool,
        *,
        clipping_norm: float | PerGroup,
        autos: bool,
        gamma: float,
        normalize_by: float,
        batch_argnums: tuple[int, ...],
        want_aux: bool,
        want_stats: bool,
        second_moment: bool,
        pre_clipping_transform: Callable,
        microbatch_size: int | None,
        dtype: torch.dtype | None,
        compute_dtype: torch.dtype | None,
        scale_fn: Callable | None,
    ) -> None:
        self.loss_fn = loss_fn
        self.argnums = argnums
        self.argnums_raw = argnums_raw
        self.has_aux = has_aux
        self.clipping_norm = clipping_norm
        self.autos = autos
        self.gamma = gamma
        self.normalize_by = float(normalize_by)
        self.batch_argnums = batch_argnums
        self.want_aux = want_aux
        self.want_stats = want_stats
        self.second_moment = second_moment
        self.transform = pre_clipping_transform
        self.microbatch_size = microbatch_size
        self.dtype = dtype
        self.compute_dtype = compute_dtype
        self.scale_fn = scale_fn
        self._discovery: tuple[tuple, _Discovery] | None = None
        # Keyword arguments for every GhostPlan this engine builds (for
        # example {"linear_pe_bytes": 0} to keep full-weight per-example
        # gradients out of HBM and take the clipped-sum GEMM instead).
        self.plan_options: dict[str, Any] = {}
        # The last plan: a call with the same structure (plan key) rebinds it
        # to its own inputs instead of building tables and buffers again.
        self._plan: GhostPlan | None = None
        self._spec_memo: tuple | None = None
        self._lora_ptrs = torch.empty(0, dtype=torch.int64)  # LoRA site addresses from plan_key
        # Host milliseconds the last call spent from its captured inputs to the
        # plan being ready (spec, plan key, rebind or build: last_prep_ms) and
        # to its last kernel enqueued (last_plan_ms), and whether it rebound
        # the previous plan.
        self.last_prep_ms = 0.0
        self.last_plan_ms = 0.0
        self.last_rebound = False
        if microbatch_size is not None and int(microbatch_size) <= 0:
            raise ValueError(f"microbatch_size must be positive, got {microbatch_size}")

    # -- helpers ---------------------------------------------------------------
    def _loss(self, *args: Any, **kwargs: Any) -> tuple[Any, Any]:
        out = self.loss_fn(*args, **kwargs)
        return out if self.has_aux else (out, ())

    def _grad_tree(self, args: tuple) -> Any:
        """The pytree torch.func.grad returns for these argnums."""
        if isinstance(self.argnums_raw, int):
            return args[self.argnums_raw]
        return tuple(args[i] for i in self.argnums)

    def _with_grad_tree(self, args: tuple, tree: Any) -> tuple:
        out = list(args)
        if isinstance(self.argnums_raw, int):
            out[self.argnums_raw] = tree
        else:
            for k, i in enumerate(self.argnums):
                out[i] = tree[k]
        return tuple(out)

    def _batch_slice(self, args: tuple, lo: int, hi: int) -> tuple:
        out = list(args)
        for i in self.batch_argnums:
            out[i] = tree_map(lambda t: t[lo:hi] if isinstance(t, torch.Tensor) else t, args[i])
        return tuple(out)

    def _in_dims(self, args: tuple, grad_in_dims: Any = None) -> tuple:
        dims = []
        for i, a in enumerate(args):
            if i in self.batch_argnums:
                dims.append(0)
            else:
                dims.append(None)
        if grad_in_dims is not None:
            if isinstance(self.argnums_raw, int):
                dims[self.argnums_raw] = grad_in_dims
            else:
                for k, i in enumerate(self.argnums):
                    dims[i] = grad_in_dims[k]
        return tuple(dims)

    def _groups(self, paths: list) -> tuple[list[int], list[str], list[float]]:
        cn = self.clipping_norm
        if not isinstance(cn, PerGroup):
            return [0] * len(paths), [], [float(cn)]
        _validate_per_group_paths(paths, cn)
        names: list[str] = []
        index: dict[str, int] = {}
        leaf_group = []
        for p in paths:
            g = cn.groups[p]
            if g not in index:
                index[g] = len(names)
                names.append(g)
            leaf_group.append(index[g])
        return leaf_group, names, [float(cn.values[g]) for g in names]

    def _clip_spec(self, shapes: list[tuple], dtypes: list[torch.dtype], thresholds: list[float],
                   normalize_by: float, capture: bool) -> tuple[ClipSpec, list[int], bool]:
        """Clip constants, per leaf its guard class (one per storage dtype), and
        whether materialised leaves square in float64."""
        acc_request = self.compute_dtype
        if capture and acc_request is not None and acc_request.is_floating_point and (
            torch.finfo(acc_request).eps < torch.finfo(torch.float32).eps
        ):
            # The seam kernels square in float32 and sum in float64, so a wider
            # request is guarded as float32 (the guard must cover the arithmetic
            # done).  Materialised leaves square in the requested dtype.
            acc_request = torch.float32
        acc, rnd = leaf_guards(shapes, dtypes, acc_request)
        cls_of: dict[torch.dtype, int] = {}
        guards = []
        leaf_cls = []
        for dt in dtypes:
            if dt not in cls_of:
                cls_of[dt] = len(guards)
                rel, ab = guard_constants(dt, rnd)
                guards.append((rel, ab, dt))
            leaf_cls.append(cls_of[dt])
        cn = self.clipping_norm
        effective = cn.effective if isinstance(cn, PerGroup) else float(cn)
        if self.scale_fn is not None:
            # The values arrive already scaled by the caller's _scale_fn; the
            # plan sums them with scale 1 (raw_values) and the clip factors
            # only supply their norms (the clipped norms), so no threshold
            # applies.
            thresholds = [float("inf")] * len(thresholds)
            effective = float("inf")
        spec = ClipSpec(
            mode=N.CLIP_AUTOS if self.autos else N.CLIP_FIXED,
            thresholds=thresholds,
            effective=float(effective),
            gamma=float(self.gamma),
            normalize_by=float(normalize_by),
            guards=guards,
        )
        return spec, leaf_cls, acc == torch.float64

    # -- discovery -------------------------------------------------------------
    def _discover(self, args: tuple, kwargs: dict, leaves: list[torch.Tensor], treedef) -> _Discovery:
        key = tuple((id(t), t.data_ptr(), tuple(t.shape), t.dtype) for t in leaves)
        if self._discovery is not None and self._discovery[0] == key:
            return self._discovery[1]
        proxies = [t.detach().requires_grad_() for t in leaves]
        pid = {id(p): k for k, p in enumerate(proxies)}
        single = list(self._with_grad_tree(args, tree_unflatten(treedef, proxies)))
        for i in self.batch_argnums:
            single[i] = tree_map(lambda t: t[0] if isinstance(t, torch.Tensor) else t, single[i])
        sess = CaptureSession(mode="discover")
        with torch.enable_grad(), sess:
            value, _ = self._loss(*single, **kwargs)
        outside = [False] * len(leaves)
        if isinstance(value, torch.Tensor) and value.requires_grad:
            grads = torch.autograd.grad(value, proxies, allow_unused=True)
            outside = [g is not None for g in grads]
        uses = [sess.uses.get(id(p), 0) for p in proxies]
        eligible = {k for k in range(len(leaves)) if uses[k] == 1 and not outside[k]}
        for a_id, b_id, w_id, bias_id in sess.pairs:
            ka, kb, kw = pid.get(a_id), pid.get(b_id), pid.get(w_id)
            kbias = pid.get(bias_id)
            trainable = [k for k in (ka, kb) if k is not None]
            if kw is not None or any(k not in eligible for k in trainable):
                # A trainable base weight, or a factor that is also needed elsewhere,
                # keeps the whole seam on the materialised route.
                eligible.difference_update(trainable)
            del kbias
        disc = _Discovery(frozenset(eligible))
        self._discovery = (key, disc)
        return disc

    # -- one (micro)batch -------------------------------------------------------
    def _run_batch(self, args: tuple, kwargs: dict, normalize_by: float,
                   out_dtype_of: Callable[[torch.dtype], torch.dtype]) -> tuple[_StepOut, list, Any]:
        tree = self._grad_tree(args)
        paths, leaves, treedef = tree_flatten_with_paths(tree)
        for p, t in zip(paths, leaves):
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"Expected tensor leaves in the differentiated arguments; got "
                                f"{type(t).__name__} at path {p!r}.")
        device = leaves[0].device if leaves else None
        if device is None or device.type != "cuda":
            raise RuntimeError(
                "opaque_amd clipping runs on the GPU: the differentiated parameters must be CUDA tensors"
            )
        N.load()
        n = batch_size_from_args(args, self.batch_argnums)
        capture_ok = (self.transform is _identity and self.scale_fn is None
                      and all(t.dtype in _KERNEL_DTYPES for t in leaves))
        if capture_ok:
            disc = self._discover(args, kwargs, leaves, treedef)
            if disc.eligible:
                res = self._run_capture(args, kwargs, n, paths, leaves, treedef, disc,
                                        normalize_by, out_dtype_of)
                if res is not None:
                    return res
        return self._run_materialised(args, kwargs, n, normalize_by, out_dtype_of)

    def _finish(self, n: int, paths: list, treedef, shapes: list, dtypes: list, device,
                sites: list[LoraSite], mats: list[MaterializedLeaf], segments: Segments,
                normalize_by: float, out_dtype_of, values, loss_aux, all_finite,
                lins: list[LinearSite] = ()) -> tuple:
        t0 = time.perf_counter()
        capture = bool(sites) or bool(lins)
        # Clip constants and output leaves depend only on the tree's shapes,
        # dtypes and paths and on the thresholds (which adaptive clipping
        # moves every step): kept from the last call when those match.
        cn = self.clipping_norm
        memo_key = (tuple(shapes), tuple(dtypes),
                    (tuple(paths), tuple(cn.groups.items()), tuple(cn.values.items()))
                    if isinstance(cn, PerGroup) else float(cn),
                    len(paths), float(normalize_by), capture)
        if self._spec_memo is None or self._spec_memo[0] != memo_key:
            leaf_group, names, thresholds = self._groups(paths)
            spec, leaf_cls, square_f64 = self._clip_spec(shapes, dtypes, thresholds, normalize_by, capture)
            outs = [LeafOut(tuple(s), out_dtype_of(dt), leaf_group[k], leaf_cls[k])
                    for k, (s, dt) in enumerate(zip(shapes, dtypes))]
            self._spec_memo = (memo_key, (names, spec, square_f64, outs, leaves_key(outs)))
        names, spec, square_f64, outs, outs_key = self._spec_memo[1]
        # The batch sum accumulates in compute_dtype when one is given
        # (_clipped_fun.py:115-134): float64 on request, float32 otherwise.
        # A caller's _scale_fn already scaled the values: they are summed as
        # they are (scale 1, non-finite entries kept), as the reference sums
        # the scale function's output (_clipped_fun.py:673-700, 777-782).
        kw = dict(second_moment=self.second_moment, square_f64=square_f64,
                  sum_f64=self.compute_dtype == torch.float64, raw_values=self.scale_fn is not None,
                  **self.plan_options)
        if self._lora_ptrs.numel() < LORA_PTRS * len(sites):
            self._lora_ptrs = torch.empty(LORA_PTRS * len(sites), dtype=torch.int64)
        key = plan_key(segments=segments, leaves=outs, clip=spec, lora_sites=sites, materialized=mats,
                       linear_sites=lins, device=device, leaves_key_=outs_key, lora_ptrs=self._lora_ptrs, **kw)
        plan = None
        if self._plan is not None and self._plan.key == key:
            plan = self._plan
            if not plan.rebind(sites, mats, list(lins), spec, key=key, lora_ptrs=self._lora_ptrs):
                plan = None
        self.last_rebound = plan is not None
        if plan is None:
            self._plan = None  # release the old plan's buffers before building
            plan = GhostPlan(segments=segments, leaves=outs, clip=spec, lora_sites=sites,
                             materialized=mats, linear_sites=list(lins), device=device, **kw)
            self._plan = plan
        self.last_prep_ms = (time.perf_counter() - t0) * 1e3
        res = plan.run()
        self.last_plan_ms = (time.perf_counter() - t0) * 1e3
        if all_finite is not None and plan.pe_views():
            all_finite = all_finite & _pe_finite(plan)
        if all_finite is not None and lins:
            all_finite = all_finite & plan.linear_finite()
        # ||scaled gradient||: per group, scale * group norm (class 0 scale).
        cn2 = (res.scales[0].float() * res.group_norms).square().sum(0).sqrt()
        step = _StepOut(
            leaves=list(res.leaves), squared=None if res.second_moment is None else list(res.second_moment),
            norms=res.norms, group_norms=res.group_norms, clipped=res.clipped,
            clipped_total=res.clipped_total, clipped_norms=cn2, values=values, loss_aux=loss_aux,
            all_finite=all_finite,
        )
        return step, names, treedef

    def _run_materialised(self, args, kwargs, n, normalize_by, out_dtype_of):
        want_finite = self.want_stats
        loss = self._loss
        transform = self.transform
        gv = torch.func.grad_and_value(loss, argnums=self.argnums_raw, has_aux=True)

        scale_fn = self.scale_fn

        def per_example(*a):
            g, (v, aux) = gv(*a, **kwargs)
            g = transform(g)
            if scale_fn is None:
                return g, v, aux
            # _clipped_fun.py:673-700: the caller's scale function returns the
            # scaled gradient and its norm record; finiteness is of the
            # unscaled gradient.
            fin = torch.ones((), dtype=torch.bool, device=v.device)
            for t in tree_flatten_with_paths(g)[1]:
                fin = fin & torch.isfinite(t).all()
            scaled, info = scale_fn(g)
            gn = getattr(info, "group_norms", None)
            return scaled, v, aux, (info.norm, gn if gn is not None else {}, fin)

        in_dims = self._in_dims(args)
        out = torch.func.vmap(per_example, in_dims=in_dims, randomness="same")(*args)
        grads, values, loss_aux = out[:3]
        paths, pe, treedef = tree_flatten_with_paths(grads)
        for p, t in zip(paths, pe):
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"per-example gradient leaf at {p!r} is not a tensor")
            if t.dtype not in _LEAF_DTYPES:
                raise TypeError(
                    "opaque_amd kernels support float32, bfloat16, float16 and float64 gradient leaves, "
                    f"got {t.dtype} at {p!r}"
                )
        all_finite = None
        if want_finite and scale_fn is None:
            all_finite = torch.ones((), dtype=torch.bool, device=pe[0].device)
            for t in pe:
                all_finite = all_finite & torch.isfinite(t).all()
        mats = [MaterializedLeaf(per_example=t.reshape(n, -1), leaf=k) for k, t in enumerate(pe)]
        shapes = [tuple(t.shape[1:]) for t in pe]
        dtypes = [t.dtype for t in pe]
        seg = Segments.padded(n, 1)
        step, names, treedef = self._finish(n, paths, treedef, shapes, dtypes, pe[0].device, [], mats, seg,
                                            normalize_by, out_dtype_of, values.detach(), loss_aux, all_finite)
        if scale_fn is not None:
            step = self._scaled_step(step, names, *out[3])
        return step, names, treedef

    def _scaled_step(self, step: _StepOut, names: list[str], norms: torch.Tensor, gnorms: dict,
                     finite: torch.Tensor) -> _StepOut:
        """Diagnostics of a call with a custom _scale_fn: the norms are the ones
        the scale function reported, the clipped norms those of the scaled
        gradients the kernels summed, and the clip counts compare the reported
        norms with the thresholds (_clipped_fun.py:472-523, 675-700)."""
        cn = self.clipping_norm
        norms = norms.detach()
        if isinstance(cn, PerGroup) and gnorms:
            gn = torch.stack([gnorms[name].detach().to(step.group_norms.dtype) for name in names])
            thr = torch.tensor([float(cn.values[name]) for name in names], dtype=gn.dtype,
                               device=gn.device).unsqueeze(1)
            clipped_mask = (gn > thr).to(torch.uint8)
        else:
            gn = norms.to(step.group_norms.dtype).unsqueeze(0).expand(step.group_norms.shape[0], -1)
            clipped_mask = (gn > float(cn.effective if isinstance(cn, PerGroup) else cn)).to(torch.uint8)
        eff = cn.effective if isinstance(cn, PerGroup) else float(cn)
        return _StepOut(
            leaves=step.leaves, squared=step.squared, norms=norms, group_norms=gn, clipped=clipped_mask,
            clipped_total=(norms > eff).to(torch.uint8), clipped_norms=step.norms, values=step.values,
            loss_aux=step.loss_aux, all_finite=finite.all() if self.want_stats else None,
        )

    def _run_capture(self, args, kwargs, n, paths, leaves, treedef, disc, normalize_by, out_dtype_of):
        device = leaves[0].device
        expanded: dict[int, torch.Tensor] = {}
        passed: list[torch.Tensor] = []
        dims: list[int | None] = []
        for k, t in enumerate(leaves):
            if k in disc.eligible:
                passed.append(t)
                dims.append(None)
            else:
                e = t.detach().unsqueeze(0).expand(n, *t.shape).requires_grad_()
                expanded[k] = e
                passed.append(e)
                dims.append(0)
        cargs = self._with_grad_tree(args, tree_unflatten(treedef, passed))
        in_dims = self._in_dims(cargs, tree_unflatten(treedef, dims))
        anchor = torch.zeros((), dtype=torch.float32, device=device, requires_grad=True)
        obj_leaf = {id(leaves[k]): k for k in disc.eligible}
        sess = CaptureSession(mode="capture", anchor=anchor, eligible=set(obj_leaf))

        def per_example(*a):
            return self._loss(*a, **kwargs)

        with torch.enable_grad(), sess:
            values, loss_aux = torch.func.vmap(per_example, in_dims=in_dims, randomness="same")(*cargs)
        recs = sess.sites
        seen: dict[int, int] = {}
        want = dict.fromkeys(disc.eligible, 1)
        for r in recs:
            for o in (r.a_obj, r.b_obj, r.w_obj):
                if o is not None and id(o) in obj_leaf:
                    k = obj_leaf[id(o)]
                    seen[k] = seen.get(k, 0) + 1
                    if r.w_index is not None:  # a stacked (MoE) weight: one record per expert
                        want[k] = leaves[k].shape[0]
        if any(seen.get(k, 0) != want[k] for k in disc.eligible):
            # The batched pass took a different route than discovery: redo it materialised.
            self._discovery = None
            return None
        if not (isinstance(values, torch.Tensor) and values.dim() == 1 and values.shape[0] == n):
            raise ValueError("the loss function must return a scalar per example")
        targets = [anchor] + [expanded[k] for k in sorted(expanded)]
        grads = torch.autograd.grad(values.sum(), targets, allow_unused=True)
        ex_grads = dict(zip(sorted(expanded), grads[1:]))

        sites: list[LoraSite] = []
        mats: list[MaterializedLeaf] = []
        rows_per_ex: dict[int, int] = {}
        for r in recs:
            if r.g is None:
                d_out = r.w_obj.shape[-2] if r.w_obj is not None else r.B.shape[1]
                r.g = torch.zeros(*r.x.shape[:-1], d_out, dtype=r.x.dtype, device=r.x.device)
            if r.segments is not None:
                continue  # MoE experts bring their own rows
            t_rows = r.x[0].numel() // r.x.shape[-1] if r.x.dim() > 1 else 1
            rows_per_ex[t_rows] = rows_per_ex.get(t_rows, 0) + 1
        seq = max(rows_per_ex, key=rows_per_ex.get) if rows_per_ex else 1
        lins: list[LinearSite] = []
        stacked: dict[int, torch.Tensor] = {}
        for r in recs:
            if r.w_obj is not None and r.segments is not None:
                kw = obj_leaf[id(r.w_obj)]
                if (r.x.dtype == r.g.dtype == leaves[kw].dtype == torch.bfloat16
                        and supports_rows(r.x) and supports_rows(r.g)):
                    lins.append(LinearSite(x=r.x, g=r.g, w_leaf=kw, segments=r.segments, index=r.w_index))
                else:
                    pe = _expert_per_example(r, leaves[kw], n)
                    stacked[kw] = pe if kw not in stacked else stacked[kw] + pe
                continue
            if r.w_obj is not None:
                kw = obj_leaf[id(r.w_obj)]
                t_rows = r.x[0].numel() // r.x.shape[-1]
                if (t_rows == seq and r.x.shape[0] == n
                        and r.x.dtype == r.g.dtype == leaves[kw].dtype == torch.bfloat16
                        and supports_rows(r.x) and supports_rows(r.g)):
                    lins.append(LinearSite(x=r.x, g=r.g, w_leaf=kw))
                else:
                    for k, pe in _site_per_example(r, None, None, leaves, kw):
                        mats.append(MaterializedLeaf(per_example=pe.reshape(n, -1), leaf=k))
                continue
            ka = obj_leaf.get(id(r.a_obj)) if r.a_obj is not None else None
            kb = obj_leaf.get(id(r.b_obj)) if r.b_obj is not None else None
            t_rows = r.x[0].numel() // r.x.shape[-1]
            kernel_ok = (
                t_rows == seq and r.x.shape[0] == n and r.x.dtype == r.g.dtype
                and r.x.dtype in _KERNEL_DTYPES and supports_rows(r.x) and supports_rows(r.g)
                and r.A.shape[1] <= 64
                and (ka is None or leaves[ka].dtype == r.x.dtype)
                and (kb is None or leaves[kb].dtype == r.x.dtype)
            )
            if kernel_ok:
                sites.append(LoraSite(x=r.x, g=r.g, A=r.A, B=r.B, scaling=r.scaling, a_leaf=ka, b_leaf=kb,
                                      a_transposed=r.a_transposed, b_transposed=r.b_transposed, v=r.v, u=r.u))
            else:
                for k, pe in _site_per_example(r, ka, kb, leaves):
                    mats.append(MaterializedLeaf(per_example=pe.reshape(n, -1), leaf=k))
        for k, pe in stacked.items():
            mats.append(MaterializedLeaf(per_example=pe.reshape(n, -1), leaf=k))
        for k, g in ex_grads.items():
            if g is None:
                g = torch.zeros((n, *leaves[k].shape), dtype=leaves[k].dtype, device=device)
            mats.append(MaterializedLeaf(per_example=g.reshape(n, -1), leaf=k))
        all_finite = None
        if self.want_stats:
            all_finite = torch.ones((), dtype=torch.bool, device=device)
            for m in mats:
                all_finite = all_finite & torch.isfinite(m.per_example).all()
        shapes = [tuple(t.shape) for t in leaves]
        dtypes = [t.dtype for t in leaves]
        seg = Segments.padded(n, seq)
        return self._finish(n, paths, treedef, shapes, dtypes, device, sites, mats, seg,
                            normalize_by, out_dtype_of, values.detach(), loss_aux, all_finite, lins)

    # -- the call ----------------------------------------------------------------
    def __call__(self, args: tuple, kwargs: dict) -> Any:
        n = batch_size_from_args(args, self.batch_argnums)
        tree = self._grad_tree(args)
        _, leaves0, _ = tree_flatten_with_paths(tree)

        def out_dtype(dt: torch.dtype) -> torch.dtype:
            return self.dtype if self.dtype is not None else dt

        if self.microbatch_size is None or self.microbatch_size >= n:
            step, names, treedef = self._run_batch(args, kwargs, self.normalize_by, out_dtype)
            result = tree_unflatten(treedef, step.leaves)
            squared = tree_unflatten(treedef, step.squared) if step.squared is not None else None
            return self._package(result, squared, [step], names, n)

        # Microbatches: each chunk's clipped sum is kept at the accumulation width
        # and the chunks are added on the device; cast and normalize_by come last.
        mb = int(self.microbatch_size)
        steps: list[_StepOut] = []
        acc: list[torch.Tensor] | None = None
        acc2: list[torch.Tensor] | None = None
        names: list[str] = []
        treedef = None
        final_dtypes: list[torch.dtype] = []

        def acc_dtype(dt: torch.dtype) -> torch.dtype:
            target = out_dtype(dt)
            return torch.promote_types(torch.promote_types(dt, torch.float32), target) \
                if dt in (torch.bfloat16, torch.float16) else torch.promote_types(dt, target)

        for lo in range(0, n, mb):
            chunk = self._batch_slice(args, lo, min(n, lo + mb))
            step, names, treedef = self._run_batch(chunk, kwargs, 1.0, acc_dtype)
            if acc is None:
                acc = [t.clone() for t in step.leaves]
                acc2 = [t.clone() for t in step.squared] if step.squared is not None else None
                final_dtypes = [out_dtype(t.dtype) for t in tree_flatten_with_paths(self._grad_tree(chunk))[1]]
            else:
                for a, t in zip(acc, step.leaves):
                    a.add_(t)
                if acc2 is not None:
                    for a, t in zip(acc2, step.squared):
                        a.add_(t)
            step.leaves, step.squared = [], None
            steps.append(step)
        del leaves0
        nb = self.normalize_by

        def fin(ts: list[torch.Tensor]) -> list[torch.Tensor]:
            out = []
            for t, dt in zip(ts, final_dtypes):
                t = t.to(dt) if t.dtype != dt else t
                out.append(t / nb if nb != 1.0 else t)
            return out

        result = tree_unflatten(treedef, fin(acc))
        squared = tree_unflatten(treedef, fin(acc2)) if acc2 is not None else None
        return self._package(result, squared, steps, names, n)

    def _package(self, result, squared, steps: list[_StepOut], names: list[str], n: int) -> Any:
        cn = self.clipping_norm
        max_norm = cn / self.normalize_by
        if self.second_moment:
            output = SecondMomentClippingOutput(
                grads=ClippedPytree(pytree=result, max_norm=max_norm),
                squared_grads=ClippedPytree(pytree=squared, max_norm=(cn * cn) / self.normalize_by),
            )
        else:
            output = clipped(result, max_norm=max_norm)
        if not (self.want_aux or self.want_stats):
            return output
        cat = (lambda xs: xs[0]) if len(steps) == 1 else (lambda xs: torch.cat(xs, dim=-1))
        norms = cat([s.norms for s in steps])
        gnorms = cat([s.group_norms for s in steps])
        per_group_mode = isinstance(cn, PerGroup)
        group_dict = {name: gnorms[g] for g, name in enumerate(names)} if per_group_mode else None
        if per_group_mode:
            clipped_mask = cat([s.clipped for s in steps])
            counts = clipped_mask.sum(dim=1, dtype=torch.int64).tolist()
            num_clipped: Any = {name: float(counts[g]) for g, name in enumerate(names)}
            rate: Any = {k: v / float(n) for k, v in num_clipped.items()} if n else dict.fromkeys(names, 0.0)
        else:
            total = int(cat([s.clipped_total for s in steps]).sum(dtype=torch.int64).item())
            num_clipped = float(total)
            rate = num_clipped / float(n) if n else 0.0
        if self.want_stats:
            finite = True
            flags = [s.all_finite for s in steps if s.all_finite is not None]
            if flags:
                finite = bool(torch.stack(flags).all().item())
            return output, ClippingStats(num_clipped=num_clipped, clipping_rate=rate, batch_size=n,
                                         all_finite=finite)
        values = cat([s.values for s in steps]) if steps[0].values is not None else None
        loss_aux = None
        if self.has_aux:
            if len(steps) == 1:
                loss_aux = steps[0].loss_aux
            else:
                loss_aux = tree_map(lambda *xs: torch.cat(xs, dim=0),
                                    steps[0].loss_aux, *[s.loss_aux for s in steps[1:]])
        aux_cls = AutoClippedGradAux if self.autos else ClippedGradAux
        aux = aux_cls(
            loss_values=values,
            grad_norms=norms,
            clipped_grad_norms=cat([s.clipped_norms for s in steps]),
            loss_aux=loss_aux,
            clipping_rate=rate if isinstance(rate, float) else None,
            batch_size=n,
            group_norms=group_dict,
        )
        return output, aux


def _pe_finite(plan: GhostPlan) -> torch.Tensor:
    """Whether the stored per-example factor gradients are all finite."""
    ok = torch.ones((), dtype=torch.bool, device=plan.device)
    for view in plan.pe_views():
        ok = ok & torch.isfinite(view).all()
    return ok


def _site_per_example(r: SiteRecord, ka: int | None, kb: int | None,
                      leaves: list[torch.Tensor], kw: int | None = None) -> list[tuple[int, torch.Tensor]]:
    """Per-example gradients of a seam the kernels cannot take, in the leaf dtype.

    dA_i = s X_i^T (G_i B^T), dB_i = s (X_i A)^T G_i (LoRA) and dW_i = G_i^T X_i
    (full-weight linear) over each example's rows.
    """
    n = r.x.shape[0]
    x = r.x.reshape(n, -1, r.x.shape[-1])
    g = r.g.reshape(n, -1, r.g.shape[-1])
    out = []
    if kw is not None:
        dt = leaves[kw].dtype
        out.append((kw, torch.matmul(g.to(dt).transpose(1, 2).contiguous(), x.to(dt))))
        return out
    if ka is not None:
        dt = leaves[ka].dtype
        u = torch.matmul(g.to(dt), r.B.to(dt).t().contiguous())  # [n, T, r]
        da = r.scaling * torch.matmul(x.to(dt).transpose(1, 2).contiguous(), u)  # [n, d_in, r]
        out.append((ka, da.transpose(1, 2) if r.a_transposed else da))
    if kb is not None:
        dt = leaves[kb].dtype
        v = torch.matmul(x.to(dt), r.A.to(dt))  # [n, T, r]
        db = r.scaling * torch.matmul(v.transpose(1, 2).contiguous(), g.to(dt))  # [n, r, d_out]
        out.append((kb, db.transpose(1, 2) if r.b_transposed else db))
    return out


def _expert_per_example(r: SiteRecord, leaf: torch.Tensor, n: int) -> torch.Tensor:
    """Per-example gradients [n, E, d_out, d_in] of one MoE expert's weight slice (others zero),
    for experts the kernels cannot take: dW_i = G_i^T X_i over example i's rows of the expert."""
    dt = leaf.dtype
    full = torch.zeros((n, *leaf.shape), dtype=dt, device=leaf.device)
    seg = r.segments
    for s, ln, ex in zip(seg.starts, seg.lengths, seg.examples):
        if ln:
            full[ex, r.w_index] = r.g[s : s + ln].to(dt).t().contiguous() @ r.x[s : s + ln].to(dt)
    return full


# ---------------------------------------------------------------------------
# Factories
# ---------------------------------------------------------------------------


def _empty_response(args, state, *, argnums, clipping_norm, normalize_by, second_moment,
                    return_aux, return_stats, aux_cls):
    """Zero gradients and empty diagnostics for a batch of size 0 (_clipped_grad.py:216-256)."""
    max_norm = clipping_norm / normalize_by
    zeros = _zero_grads_like(args, argnums)
    if second_moment:
        grads: Any = SecondMomentClippingOutput(
            grads=clipped(zeros, max_norm=max_norm),
            squared_grads=clipped(_zero_grads_like(args, argnums),
                                  max_norm=(clipping_norm * clipping_norm) / normalize_by),
        )
    else:
        grads = clipped(zeros, max_norm=max_norm)
    if return_aux:
        empty = torch.empty(0)
        aux = aux_cls(loss_values=empty, grad_norms=empty, clipped_grad_norms=empty, loss_aux=None,
                      clipping_rate=0.0, batch_size=0)
        return (grads, aux), state
    if return_stats:
        if isinstance(clipping_norm, PerGroup):
            stats = ClippingStats(num_clipped=dict.fromkeys(clipping_norm.values, 0.0),
                                  clipping_rate=dict.fromkeys(clipping_norm.values, 0.0), batch_size=0)
        else:
            stats = ClippingStats(num_clipped=0.0, clipping_rate=0.0, batch_size=0)
        return (grads, stats), state
    return grads, state


def under_differentiating_transform() -> bool:
    """Whether an enclosing torch.func grad, vjp or jvp is active (the
    reference's test, ``ENG/functional/_transform_stack.py:10-21``)."""
    try:
        from torch._C._functorch import TransformType, get_interpreter_stack
    except ImportError:  # pragma: no cover - the functorch C API moved
        return False
    stack = get_interpreter_stack() or ()
    return any(i.key() in (TransformType.Grad, TransformType.Jvp) for i in stack)


def _make(loss_fn, argnums, has_aux, *, clipping_norm, autos, gamma, normalize_by, batch_argnums,
          return_aux, return_stats, second_moment, pre_clipping_transform, microbatch_size, dtype,
          compute_dtype, scale_fn, aux_cls, label):
    argnums_t = _to_tuple(argnums)
    batch_t = _to_tuple(batch_argnums)
    engine = _ClipEngine(
        loss_fn, argnums_t, argnums, has_aux, clipping_norm=clipping_norm, autos=autos, gamma=gamma,
        normalize_by=normalize_by, batch_argnums=batch_t, want_aux=return_aux, want_stats=return_stats,
        second_moment=second_moment, pre_clipping_transform=pre_clipping_transform,
        microbatch_size=microbatch_size, dtype=dtype, compute_dtype=compute_dtype, scale_fn=scale_fn,
    )

    def grad_fn(*args, state, **kwargs):
        if batch_size_from_args(args, batch_t) == 0:
            return _empty_response(args, state, argnums=argnums_t, clipping_norm=clipping_norm,
                                   normalize_by=normalize_by, second_moment=second_moment,
                                   return_aux=return_aux, return_stats=return_stats, aux_cls=aux_cls)
        # The reference keeps the graph for an enclosing grad/jvp
        # (_clipped_grad.py:261-265); the clip and sum kernels here have no
        # derivative, so such a call is refused rather than silently detached.
        if under_differentiating_transform():
            raise NotImplementedError(
                f"{label.split('::')[-1]} cannot run under an enclosing torch.func grad/vjp/jvp: its clip and sum "
                "kernels are not differentiable (call it outside the transform)")
        with record_function(label):
            out = engine(args, kwargs)
        return out, state

    grad_fn.engine = engine  # type: ignore[attr-defined]
    return grad_fn


def clipped_grad(
    loss_fn: Callable,
    argnums: int | tuple[int, ...] = 0,
    has_aux: bool = False,
    *,
    clipping_norm: float | PerGroup,
    normalize_by: float = 1.0,
    batch_argnums: int | tuple[int, ...] = 1,
    return_aux: bool = False,
    return_stats: bool = False,
    second_moment: bool = False,
    pre_clipping_transform: Callable = _identity,
    microbatch_size: int | None = None,
    dtype: torch.dtype | None = None,
    compute_dtype: torch.dtype | None = None,
    _scale_fn: Callable | None = None,
) -> tuple[Callable, FixedClipState]:
    """Sum of per-example gradients clipped to ``clipping_norm`` (``_clipped_grad.py:81-341``).

    Returns ``(grad_fn, FixedClipState())``; ``grad_fn(*args, state=...)``
    returns ``(ClippedPytree(sum / normalize_by, max_norm=C / normalize_by), state)``,
    or ``((grads, ClippedGradAux), state)`` with ``return_aux``, or
    ``((grads, ClippingStats), state)`` with ``return_stats``.
    """
    _validate_static_args(argnums, batch_argnums, normalize_by)
    if return_aux and return_stats:
        raise ValueError("return_stats cannot be combined with return_aux=True")
    _validate_clipping_norm(clipping_norm)
    if compute_dtype is not None and not compute_dtype.is_floating_point:
        raise TypeError(f"compute_dtype must be a real floating-point dtype, got {compute_dtype!r}.")
    fn = _make(loss_fn, argnums, has_aux, clipping_norm=clipping_norm, autos=False, gamma=0.0,
               normalize_by=normalize_by, batch_argnums=batch_argnums, return_aux=return_aux,
               return_stats=return_stats, second_moment=second_moment,
               pre_clipping_transform=pre_clipping_transform, microbatch_size=microbatch_size,
               dtype=dtype, compute_dtype=compute_dtype, scale_fn=_scale_fn, aux_cls=ClippedGradAux,
               label="opaque::clipped_grad")
    return fn, FixedClipState()


def auto_clipped_grad(
    loss_fn: Callable,
    argnums: int | tuple[int, ...] = 0,
    has_aux: bool = False,
    *,
    R: float | PerGroup = 1.0,
    gamma: float = _DEFAULT_GAMMA,
    normalize_by: float = 1.0,
    batch_argnums: int | tuple[int, ...] = 1,
    return_aux: bool = False,
    return_stats: bool = False,
    pre_clipping_transform: Callable = _identity,
    microbatch_size: int | None = None,
    dtype: Any = None,
    second_moment: bool = False,
) -> tuple[Callable, AutoClipState]:
    """Sum of AUTO-S scaled per-example gradients ``R g_i / (||g_i|| + gamma)`` (``_auto.py:200-354``).

    ``max_norm`` of the result is ``R / normalize_by``.
    """
    _validate_auto_params(R, gamma)
    _validate_static_args(argnums, batch_argnums, normalize_by)
    if return_aux and return_stats:
        raise ValueError("return_stats cannot be combined with return_aux=True")
    fn = _make(loss_fn, argnums, has_aux, clipping_norm=R, autos=True, gamma=gamma,
               normalize_by=normalize_by, batch_argnums=batch_argnums, return_aux=return_aux,
               return_stats=return_stats, second_moment=second_moment,
               pre_clipping_transform=pre_clipping_transform, microbatch_size=microbatch_size,
               dtype=dtype, compute_dtype=None, scale_fn=None, aux_cls=AutoClippedGradAux,
               label="opaque::clipped_grad")
    return fn, AutoClipState()


__all__ = [
    "AutoClipState",
    "AutoClippedGradAux",
    "ClippedGradAux",
    "ClippingStats",
    "FixedClipState",
    "auto_clipped_grad",
    "batch_size_from_args",
    "clipped_grad",
    "per_group",
]
