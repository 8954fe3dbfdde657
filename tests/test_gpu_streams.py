"""The projection and factor stages run their launches side by side on
forked streams (one per table: rank blocks of different activations).  Each
launch writes its own planes, per-example gradients and partial slots, so
the concurrent schedule must give the same bits as one launch at a time on
the caller's stream, on every run."""

from __future__ import annotations

import math

import pytest
import torch

from opaque_amd import _native as N
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LoraSite, Segments
from opaque_amd.guard import guard_constants, leaf_guards

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer_plan(seed=0):
    """One Llama-like layer at small widths: q/k/v share x (three rank blocks),
    gate/up share h (two), o alone (one), down mirrored (d_in > d_out)."""
    g = torch.Generator().manual_seed(seed)
    n_ex, T, r, d = 5, 96, 16, 256
    lengths = [96, 33, 1, 70, 64]
    shapes = {"q": (d, d), "k": (d, 64), "v": (d, 64), "o": (d, d), "gate": (d, 704), "up": (d, 704),
              "down": (704, d)}
    acts = {"x": d, "a": d, "h": d, "m": 704}
    src = {"q": "x", "k": "x", "v": "x", "o": "a", "gate": "h", "up": "h", "down": "m"}
    X = {k: torch.randn(n_ex * T, w, generator=g).to(torch.bfloat16).to(DEV) for k, w in acts.items()}
    sites, leaves, lshape = [], [], []
    for name, (d_in, d_out) in shapes.items():
        G = torch.randn(n_ex * T, d_out, generator=g).to(torch.bfloat16).to(DEV)
        A = (torch.randn(d_in, r, generator=g) / math.sqrt(d_in)).to(torch.bfloat16).to(DEV)
        B = (torch.randn(r, d_out, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
        ia, ib = len(leaves), len(leaves) + 1
        leaves += [LeafOut(tuple(A.shape), torch.bfloat16), LeafOut(tuple(B.shape), torch.bfloat16)]
        lshape += [tuple(A.shape), tuple(B.shape)]
        sites.append(LoraSite(X[src[name]], G, A, B, 2.0, a_leaf=ia, b_leaf=ib))
    _, rnd = leaf_guards(lshape, [torch.bfloat16] * len(lshape))
    rel, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[1.0], effective=1.0, normalize_by=float(n_ex),
                    guards=[(rel, ab, torch.bfloat16)])
    seg = Segments.padded(n_ex, T, lengths)
    return GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=sites, device=DEV)


def _snapshot(res):
    return [t.clone() for t in res.leaves] + [res.norms.clone(), res.scales.clone()]


def test_concurrent_stages_equal_serial_bit_for_bit():
    print("streams: one small layer, serial vs forked project/factor stages", flush=True)
    plan = _layer_plan()
    tables = [i[0] for i in plan.launch_info]
    assert tables.count("project") >= 2 and tables.count("factor") >= 2, tables
    runs = {}
    for serial in (True, False, True, False):
        plan.serial = serial
        snap = _snapshot(plan.run())
        torch.cuda.synchronize()
        runs.setdefault(serial, []).append(snap)
    want = runs[True][0]
    assert all(torch.isfinite(t.float()).all() for t in want)
    for snaps in runs.values():
        for snap in snaps:
            for a, b in zip(snap, want):
                assert torch.equal(a, b)
