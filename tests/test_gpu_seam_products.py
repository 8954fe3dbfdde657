"""LoRA sites that bring the seam's own rank-space products.

The LoRA seam computes V = x A in its forward and U = g B^T for the input
gradient in its backward (the reference's merged dX forms the same
grad_out @ B.t(), opaque-patches/.../kernels/lora.py:157-160).  A plan whose
sites bring both lays them out as planes (odp_pack_planes) and runs only the
factor kernels: one pass over X for every site's dA and one over each G for
its dB, instead of projecting X and G again.

Given the very planes the projection kernels wrote (GhostPlan.rank_planes of
a plan without products), the factor kernels see the same inputs, so every
output must be bit-identical to the projecting plan's: clipped sums, norms,
scales and masks.  Covered: activations shared by three sites (one factor
frozen), a down projection (the mirrored order without products), ragged
and empty segments, fp32, MoE-style per-site segments, and second moments.
"""

from __future__ import annotations

import math

import pytest
import torch

from opaque_amd import _native as N
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LoraSite, Segments
from opaque_amd.guard import guard_constants, leaf_guards

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(kind: str, seed: int = 0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    dt = torch.float32 if kind == "fp32" else torch.bfloat16
    n_ex, T = 4, 96
    seg = Segments.padded(n_ex, T, [96, 0, 41, 77])
    n_rows = n_ex * T

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, device=DEV, generator=g) * scale).to(dt)

    sites, leaves = [], []

    def add(x, d_out, r, frozen=(), segments=None, rows=n_rows):
        d_in = x.shape[-1]
        A = rnd(d_in, r, scale=1 / math.sqrt(d_in))
        B = rnd(r, d_out, scale=0.05)
        ia = ib = None
        if "A" not in frozen:
            ia = len(leaves)
            leaves.append(LeafOut((d_in, r), dt))
        if "B" not in frozen:
            ib = len(leaves)
            leaves.append(LeafOut((r, d_out), dt))
        sites.append(LoraSite(x, rnd(rows, d_out, scale=0.3), A, B, 2.0, a_leaf=ia, b_leaf=ib, segments=segments))

    if kind in ("qkv", "fp32", "second"):
        x = rnd(n_rows, 256)
        add(x, 256, 16)
        add(x, 64, 16, frozen=("A",))
        add(x, 64, 8)
    if kind in ("down", "second"):
        add(rnd(n_rows, 512), 128, 16)  # wider input than output: mirrored when projecting
    if kind == "moe":
        # Two experts, each with its own rows and one segment per example.
        for lens in ([30, 0, 12, 50], [7, 19, 0, 33]):
            starts = [sum(lens[:i]) for i in range(n_ex)]
            rows = sum(lens)
            es = Segments(starts, lens, list(range(n_ex)), n_ex, rows)
            add(rnd(rows, 128), 192, 16, segments=es, rows=rows)
    return seg, sites, leaves, dt


def _plan(seg, sites, leaves, dt, second=False):
    shapes = [lf.shape for lf in leaves]
    _, rnd = leaf_guards(shapes, [dt] * len(shapes))
    rel, ab = guard_constants(dt, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[0.4], effective=0.4, normalize_by=4.0, guards=[(rel, ab, dt)])
    return GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=sites, device=DEV, second_moment=second)


def _outputs(res):
    out = [t.clone() for t in res.leaves] + [res.norms.clone(), res.scales.clone(), res.clipped.clone()]
    return out + [t.clone() for t in (res.second_moment or [])]


@pytest.mark.parametrize("kind", ["qkv", "down", "fp32", "moe", "second"])
def test_seam_products_equal_projected_planes(kind):
    print(f"seam products: {kind}", flush=True)
    seg, sites, leaves, dt = _case(kind)
    second = kind == "second"
    base = _plan(seg, sites, leaves, dt, second)
    live = {t[0] for t in base.tables if t[5] > 0}
    assert "planes" not in live and "project" in live
    want = _outputs(base.run())
    torch.cuda.synchronize()
    with_vu = []
    for i, s in enumerate(sites):
        v, u = base.rank_planes(i)
        with_vu.append(LoraSite(s.x, s.g, s.A, s.B, s.scaling, a_leaf=s.a_leaf, b_leaf=s.b_leaf,
                                segments=s.segments, v=v.contiguous(), u=u.contiguous()))
    plan = _plan(seg, with_vu, leaves, dt, second)
    live = {t[0] for t in plan.tables if t[5] > 0}
    assert "planes" in live and not live & {"project", "factor_project", "pack"}, live
    got = _outputs(plan.run())
    torch.cuda.synchronize()
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), k
    # The planes the products plan laid out equal the projected ones on every
    # row of a segment (rows outside the segments are 0 here).
    for i, s in enumerate(with_vu):
        segs = s.segments if s.segments is not None else seg
        rows = torch.cat([torch.arange(st, st + ln) for st, ln in zip(segs.starts, segs.lengths)]).to(DEV)
        for mine, theirs in zip(plan.rank_planes(i), (s.v, s.u)):
            assert torch.equal(mine[rows], theirs[rows]), i
