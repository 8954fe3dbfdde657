"""Register this package under the reference's import paths.

After ``opaque_amd.alias.install()``, code written against the reference
keeps its imports: ``opaque.dpsgd.clipping`` (``clipped_grad``,
``auto_clipped_grad``, ``per_group``), ``opaque.dpsgd.noise``
(``gaussian_noise``), ``opaque.types``, ``opaque.random`` and
``opaque.pytree`` (the public modules of ``opaque-dpsgd`` and
``opaque-engine``, README.md:26-28 of the reference) resolve to the
MI355X implementation.  Nothing is installed on import; an ``opaque``
package that is already importable is left alone unless ``force=True``.
"""

from __future__ import annotations

import importlib.util
import sys
import types

from opaque_amd import adaptive, clipping, noise, pytree, random, types as dp_types

_MODULES = {
    "opaque.types": (dp_types, ["PerGroup", "ClippedPytree", "NoisedPytree", "ClipState", "NoiseState",
                                "SecondMomentClippingOutput", "SecondMomentNoiseOutput", "ParamPath",
                                "clipped", "noised"]),
    "opaque.random": (random, ["RngKey", "key", "fold_in", "split", "generator_from_key", "random_key"]),
    "opaque.pytree": (pytree, ["ParamPath", "param_path", "param_path_display", "tree_flatten",
                               "tree_flatten_with_paths", "tree_unflatten", "tree_map", "tree_map_with_path",
                               "tree_leaves", "tree_structure", "global_norm"]),
    "opaque.dpsgd.clipping": (clipping, ["clipped_grad", "auto_clipped_grad", "per_group"]),
    "opaque.dpsgd.clipping.adaptive": (adaptive, ["adaptive_clipped_grad", "AdaptiveClipState",
                                                  "AdaptiveClippedGradAux"]),
    "opaque.dpsgd.clipping.types": (clipping, ["FixedClipState", "AutoClipState", "ClippedGradAux",
                                               "AutoClippedGradAux", "ClippingStats"]),
    "opaque.dpsgd.noise": (noise, ["gaussian_noise"]),
    "opaque.dpsgd.noise.types": (noise, ["GaussianNoiseState"]),
}


def install(force: bool = False) -> bool:
    """Create the ``opaque.*`` modules in ``sys.modules``; returns whether it did."""
    if not force and ("opaque" in sys.modules or importlib.util.find_spec("opaque") is not None):
        return False
    made: dict[str, types.ModuleType] = {}

    def module(name: str) -> types.ModuleType:
        if name in made:
            return made[name]
        mod = types.ModuleType(name, f"opaque_amd implementation of {name}")
        mod.__path__ = []  # a package, so submodules can hang below it
        made[name] = mod
        sys.modules[name] = mod
        if "." in name:
            parent, _, child = name.rpartition(".")
            setattr(module(parent), child, mod)
        return mod

    for name, (src, names) in _MODULES.items():
        mod = module(name)
        for attr in names:
            setattr(mod, attr, getattr(src, attr))
        mod.__all__ = list(names)
    module("opaque.dpsgd.clipping").adaptive_clipped_grad = adaptive.adaptive_clipped_grad
    types_mod = module("opaque.dpsgd.clipping.types")
    types_mod.AdaptiveClipState = adaptive.AdaptiveClipState
    types_mod.AdaptiveClippedGradAux = adaptive.AdaptiveClippedGradAux
    dpsgd = module("opaque.dpsgd")
    dpsgd.adaptive_clipped_grad = adaptive.adaptive_clipped_grad
    for attr in ("clipped_grad", "auto_clipped_grad", "per_group"):
        setattr(dpsgd, attr, getattr(clipping, attr))
    dpsgd.gaussian_noise = noise.gaussian_noise
    return True


__all__ = ["install"]
