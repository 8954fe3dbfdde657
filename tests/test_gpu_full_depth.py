"""Whole-model plans at their configured depth and batch.

C3: the plan bench.py times -- 32 Llama-3-8B layers of LoRA r16 (448 leaves,
47k partial slots per example), batch 16 x 1024 with ragged lengths, AUTO-S,
the sites bringing the seam's V and U (bench.c3_sites builds the very same
inputs).  C2: 12 GPT-2-small layers of LoRA r8, batch 64 x 512, per-example
output-gradient scales LogNormal(0, 1), fixed clipping; V and U projected in
the step.

Each plan is checked against per-example factor gradients formed in plain
fp32 on the device (bmm over the padded batch, padding rows masked): norms
rel 2e-2, clipped sums rel 2e-2 per leaf, and the kernel's per-example clip
masks equal away from the 1e-3 band after rebinding to a threshold at the
median norm (so both outcomes occur).  The fp32 reference is itself checked
against the fp64 CPU oracle (oracle/lora_ref) on one example of one site.
"""

from __future__ import annotations

import math
from dataclasses import replace

import pytest
import torch

import bench
from opaque_amd import _native as N
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LoraSite, Segments
from opaque_amd.guard import guard_constants, leaf_guards
from oracle import lora_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _reference(sites, seg, T, scaling=2.0):
    """Per-example fp32 (dA [B, d_in, r], dB [B, r, d_out]) per site and the
    squared norms [B] (fp64, CPU)."""
    B = seg.n_ex
    mask = torch.zeros(B, T, 1, device=DEV)
    for i, ln in enumerate(seg.lengths):
        mask[i, :ln] = 1.0
    pes, sq = [], torch.zeros(B, dtype=torch.float64, device=DEV)
    for s in sites:
        x = s.x.float().view(B, T, -1) * mask
        g = s.g.float().view(B, T, -1) * mask
        dA = scaling * torch.bmm(x.transpose(1, 2).contiguous(), torch.matmul(g, s.B.float().t()))
        dB = scaling * torch.bmm(torch.matmul(x, s.A.float()).transpose(1, 2).contiguous(), g)
        del x, g
        sq += dA.double().square().sum((1, 2)) + dB.double().square().sum((1, 2))
        pes.append((dA, dB))
    return pes, sq.cpu()


def _check(plan, res, sites, pes, norms, *, autos, C, gamma, normalize_by):
    assert torch.allclose(res.norms.double().cpu(), norms, rtol=2e-2, atol=0), \
        ((res.norms.double().cpu() / norms) - 1).abs().max()
    fac = (C / (norms + gamma)) if autos else torch.clamp(C / norms, max=1.0)
    fac = fac.to(DEV).view(-1, 1, 1)
    for k, (s, (dA, dB)) in enumerate(zip(sites, pes)):
        for leaf, pe in ((s.a_leaf, dA), (s.b_leaf, dB)):
            want = (fac * pe).sum(0) / normalize_by
            got = res.leaves[leaf].float()
            err = ((got - want).norm() / want.norm()).item()
            assert err <= 2e-2, (k, leaf, err)


def _masks(plan, sites, clip, norms, C):
    """Rebinds the plan to the same inputs with threshold C and compares the
    kernel's per-example masks with norm > C away from the band."""
    assert plan.rebind(sites, [], [], replace(clip, thresholds=[C], effective=C))
    res = plan.run()
    torch.cuda.synchronize()
    far = ((norms - C).abs() / C) > 1e-3
    got = res.clipped_total.cpu().bool()
    assert torch.equal(got[far], (norms > C)[far]), (got, norms, C)
    assert 0 < int((norms > C).sum()) < len(norms)


def _oracle_spot_check(site, seg, pes, j=0):
    """The fp32 device reference against the fp64 CPU oracle, example j."""
    st, ln = seg.starts[j], seg.lengths[j]
    dA, dB = lora_ref.lora_per_example(site.x[st : st + ln].cpu(), site.g[st : st + ln].cpu(), site.A.cpu(),
                                       site.B.cpu(), 2.0, [0], [ln])
    for mine, ref in zip((pes[0][j], pes[1][j]), (dA[0], dB[0])):
        assert (mine.double().cpu() - ref).norm() <= 1e-4 * ref.norm()


def test_full_c3_plan_as_benched():
    print("full depth: C3, 32 layers, the bench's inputs and plan", flush=True)
    B, T, r = 16, 1024, 16
    seg, lengths, sites, leaves, (rel, ab) = bench.c3_sites(32, B, T, r, seed=0, seam=True, dev=DEV)
    assert len(sites) == 224 and len(leaves) == 448
    clip = ClipSpec(mode=N.CLIP_AUTOS, thresholds=[1.0], effective=1.0, gamma=0.01, normalize_by=float(B),
                    guards=[(rel, ab, torch.bfloat16)])
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=sites, device=DEV)
    live = {t[0] for t in plan.tables if t[5] > 0}
    assert "planes" in live and not live & {"project", "factor_project"}, live
    res = plan.run()
    torch.cuda.synchronize()
    pes, sq = _reference(sites, seg, T)
    norms = sq.sqrt()
    _oracle_spot_check(sites[6], seg, pes[6])  # layer 0's down projection
    _check(plan, res, sites, pes, norms, autos=True, C=1.0, gamma=0.01, normalize_by=float(B))
    _masks(plan, sites, clip, norms, float(norms.median()))


def test_full_c2_plan():
    print("full depth: C2, 12 layers, batch 64 x 512", flush=True)
    B, T, r = 64, 512, 8
    shapes = {"q": (768, 768), "k": (768, 768), "v": (768, 768), "o": (768, 768), "fc": (768, 3072),
              "proj": (3072, 768)}
    shared = {"k": "q", "v": "q"}
    g = torch.Generator(device=DEV).manual_seed(12)
    scale = torch.exp(torch.randn(B, device=DEV, generator=g)).repeat_interleave(T).view(-1, 1) * 0.02
    seg = Segments.padded(B, T)
    sites, leaves, lshapes = [], [], []
    for _ in range(12):
        xs = {}
        for name, (d_in, d_out) in shapes.items():
            key = shared.get(name, name)
            if key not in xs:
                xs[key] = torch.randn(B * T, d_in, device=DEV, generator=g).to(torch.bfloat16)
            gt = (torch.randn(B * T, d_out, device=DEV, generator=g) * scale).to(torch.bfloat16)
            A = (torch.randn(d_in, r, device=DEV, generator=g) / math.sqrt(d_in)).to(torch.bfloat16)
            Bm = (torch.randn(r, d_out, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
            ia = len(leaves)
            leaves += [LeafOut((d_in, r), torch.bfloat16), LeafOut((r, d_out), torch.bfloat16)]
            lshapes += [(d_in, r), (r, d_out)]
            sites.append(LoraSite(xs[key], gt, A, Bm, 2.0, a_leaf=ia, b_leaf=ia + 1))
    assert len(leaves) == 144
    pes, sq = _reference(sites, seg, T)
    norms = sq.sqrt()
    C = float(norms.median())
    _, rnd = leaf_guards(lshapes, [torch.bfloat16] * len(lshapes))
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[C], effective=C, normalize_by=float(B),
                    guards=[(*guard_constants(torch.bfloat16, rnd), torch.bfloat16)])
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=sites, device=DEV)
    live = {t[0] for t in plan.tables if t[5] > 0}
    assert "project" in live and "planes" not in live, live
    res = plan.run()
    torch.cuda.synchronize()
    _oracle_spot_check(sites[5], seg, pes[5], j=3)  # layer 0's proj (3072 -> 768)
    _check(plan, res, sites, pes, norms, autos=False, C=C, gamma=0.0, normalize_by=float(B))
    far = ((norms - C).abs() / C) > 1e-3
    assert torch.equal(res.clipped_total.cpu().bool()[far], (norms > C)[far])
    assert 0 < int((norms > C).sum()) < B
