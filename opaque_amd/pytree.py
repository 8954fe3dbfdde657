"""Pytree traversal with the leaf order and paths of the reference.

The reference wraps optree (``opaque-engine/.../engine/pytree.py:67-152``):
dict keys are visited in sorted order, sequences by index, ``None`` is an
empty node, and a leaf's path (``ParamPath``) is the tuple of keys/indices
leading to it.  That order fixes the summation order of norms, the PerGroup
path keys and the noise stream assignment, so it is kept exactly; the
implementation here is self-contained (no optree dependency).
"""

from __future__ import annotations

from collections import OrderedDict, defaultdict
from collections.abc import Callable
from dataclasses import dataclass
from typing import Any

import torch

ParamPath = tuple  # tuple[str | int, ...]


def param_path(path: Any) -> ParamPath:
    """Normalise a path (or a flat string key) to a tuple of str/int parts."""
    if isinstance(path, str):
        return (path,)
    out = []
    for part in path:
        if isinstance(part, (str, int)):
            out.append(part)
        else:
            raise TypeError(f"ParamPath components must be str or int; got {type(part).__name__}")
    return tuple(out)


def param_path_display(path: ParamPath) -> str:
    """Dotted display form used for pattern matching and messages."""
    return ".".join(str(p) for p in path)


def _is_namedtuple(x: Any) -> bool:
    return isinstance(x, tuple) and hasattr(type(x), "_fields")


def _sorted_keys(d: dict) -> list:
    try:
        return sorted(d.keys())
    except TypeError:
        return sorted(d.keys(), key=lambda k: (type(k).__name__, repr(k)))


@dataclass(frozen=True)
class TreeDef:
    """Structure of a pytree: node kind, node metadata and child structures."""

    kind: str  # "leaf" | "none" | "dict" | "odict" | "ddict" | "list" | "tuple" | "ntuple"
    meta: Any
    children: tuple

    @property
    def num_leaves(self) -> int:
        if self.kind == "leaf":
            return 1
        return sum(c.num_leaves for c in self.children)


_LEAF = TreeDef("leaf", None, ())


def _flatten(tree: Any, path: tuple, paths: list, leaves: list) -> TreeDef:
    if tree is None:
        return TreeDef("none", None, ())
    if isinstance(tree, (OrderedDict, defaultdict, dict)) and not isinstance(tree, torch.Tensor):
        if isinstance(tree, OrderedDict):
            keys, kind, meta = list(tree.keys()), "odict", None
        elif isinstance(tree, defaultdict):
            keys, kind, meta = _sorted_keys(tree), "ddict", (tree.default_factory, list(tree.keys()))
        else:
            keys, kind, meta = _sorted_keys(tree), "dict", list(tree.keys())
        kids = tuple(_flatten(tree[k], path + (k,), paths, leaves) for k in keys)
        return TreeDef(kind, (keys, meta), kids)
    if _is_namedtuple(tree):
        kids = tuple(_flatten(v, path + (i,), paths, leaves) for i, v in enumerate(tree))
        return TreeDef("ntuple", type(tree), kids)
    if isinstance(tree, (list, tuple)):
        kids = tuple(_flatten(v, path + (i,), paths, leaves) for i, v in enumerate(tree))
        return TreeDef("list" if isinstance(tree, list) else "tuple", None, kids)
    paths.append(path)
    leaves.append(tree)
    return _LEAF


def tree_flatten_with_paths(tree: Any) -> tuple[list[ParamPath], list[Any], TreeDef]:
    paths: list = []
    leaves: list = []
    td = _flatten(tree, (), paths, leaves)
    return [param_path(p) for p in paths], leaves, td


def tree_flatten(tree: Any) -> tuple[list[Any], TreeDef]:
    _, leaves, td = tree_flatten_with_paths(tree)
    return leaves, td


def _unflatten(td: TreeDef, it) -> Any:
    k = td.kind
    if k == "leaf":
        return next(it)
    if k == "none":
        return None
    vals = [_unflatten(c, it) for c in td.children]
    if k in ("dict", "odict", "ddict"):
        keys, meta = td.meta
        by_key = dict(zip(keys, vals))
        if k == "odict":
            return OrderedDict((kk, by_key[kk]) for kk in keys)
        if k == "ddict":
            factory, order = meta
            out = defaultdict(factory)
            for kk in order:
                out[kk] = by_key[kk]
            return out
        return {kk: by_key[kk] for kk in meta}  # original insertion order
    if k == "list":
        return vals
    if k == "tuple":
        return tuple(vals)
    if k == "ntuple":
        return td.meta(*vals)
    raise ValueError(f"unknown node kind {k}")


def tree_unflatten(treedef: TreeDef, leaves: list[Any]) -> Any:
    it = iter(leaves)
    out = _unflatten(treedef, it)
    rest = list(it)
    if rest:
        raise ValueError(f"tree_unflatten got {len(rest)} extra leaves")
    return out


def tree_structure(tree: Any) -> TreeDef:
    return tree_flatten(tree)[1]


def tree_leaves(tree: Any) -> list[torch.Tensor]:
    """Tensor leaves in traversal order (non-tensor leaves are skipped)."""
    return [x for x in tree_flatten(tree)[0] if isinstance(x, torch.Tensor)]


def tree_map(fn: Callable[..., Any], tree: Any, *rest: Any) -> Any:
    leaves, td = tree_flatten(tree)
    others = []
    for r in rest:
        rl, rtd = tree_flatten(r)
        if len(rl) != len(leaves):
            raise ValueError("tree_map: pytrees have different structures")
        others.append(rl)
    return tree_unflatten(td, [fn(x, *(o[i] for o in others)) for i, x in enumerate(leaves)])


def tree_map_with_path(fn: Callable[[ParamPath, Any], Any], tree: Any) -> Any:
    paths, leaves, td = tree_flatten_with_paths(tree)
    return tree_unflatten(td, [fn(p, x) for p, x in zip(paths, leaves)])


def global_norm(tree: Any, *, compute_dtype: torch.dtype | None = None) -> torch.Tensor:
    """sqrt(sum ||leaf||^2) with bf16/fp16 promoted to float32 (ENG/pytree.py:336-430)."""
    if compute_dtype is not None and not compute_dtype.is_floating_point:
        raise TypeError(f"compute_dtype must be a real floating-point dtype, got {compute_dtype!r}.")
    leaves = tree_leaves(tree)
    if not leaves:
        return torch.tensor(0.0, dtype=compute_dtype or torch.float32)
    if compute_dtype is not None:
        acc = compute_dtype
    else:
        acc = torch.float32
        for t in leaves:
            if t.is_floating_point():
                acc = torch.promote_types(acc, t.dtype)
            elif t.is_complex():
                acc = torch.promote_types(acc, t.real.dtype)
    total = torch.zeros((), device=leaves[0].device, dtype=acc)
    for t in leaves:
        if t.is_complex():
            re, im = t.real.to(acc), t.imag.to(acc)
            total = total + (re * re).sum(dtype=acc) + (im * im).sum(dtype=acc)
        else:
            x = t.to(acc)
            total = total + (x * x).sum(dtype=acc)
    return torch.sqrt(total)


__all__ = [
    "ParamPath",
    "TreeDef",
    "global_norm",
    "param_path",
    "param_path_display",
    "tree_flatten",
    "tree_flatten_with_paths",
    "tree_leaves",
    "tree_map",
    "tree_map_with_path",
    "tree_structure",
    "tree_unflatten",
]
