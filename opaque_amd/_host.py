"""The host-side helper extension (``csrc/odp_host.cpp``): structure
signatures and addresses of a call's LoRA sites, and output leaf views, for
GhostPlan.rebind.  Built by ``opaque_amd.build.build_host``; without it the
same work runs in Python (host bookkeeping only, no arithmetic)."""

from __future__ import annotations

import importlib.machinery
import importlib.util
from types import ModuleType

from opaque_amd.build import HOST_DIR, HOST_NAME

_mod: ModuleType | None = None
_tried = False


def load() -> ModuleType | None:
    """The helper module, or None when it has not been built."""
    global _mod, _tried
    if _tried:
        return _mod
    _tried = True
    path = HOST_DIR / f"{HOST_NAME}.so"
    if not path.exists():
        return None
    import torch  # noqa: F401  (the extension links against libtorch)

    loader = importlib.machinery.ExtensionFileLoader(HOST_NAME, str(path))
    spec = importlib.util.spec_from_loader(HOST_NAME, loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    _mod = mod
    return _mod
