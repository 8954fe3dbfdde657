"""The single-pass G side of LoRA sites (odp_seg_factor_project) against the
two-kernel path (odp_project + odp_seg_factor) and the CPU oracle.  A
one-site activation wider than its output gradient takes the mirrored
order instead (U from G first, then V and dA in one fused pass over X,
then dB), also compared bit for bit with the two-kernel path.

Both paths accumulate U = G B^T over G's columns and the dB rows over the
segment's tokens in the same order of 32-wide MFMA blocks, so their results
are compared bit for bit; the oracle comparison uses the bf16 tolerance.
"""

from __future__ import annotations

import math

import pytest
import torch

from opaque_amd import _native as N
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LoraSite, Segments
from opaque_amd.guard import guard_constants, leaf_guards
from oracle import lora_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _sites(n_rows, d_in, outs, ranks, frozen=(), seed=0):
    """Sites sharing one X; `frozen` names (site, 'A'|'B') factors without a leaf."""
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(n_rows, d_in, generator=g).to(torch.bfloat16)
    sites, leaves, shapes = [], [], []
    for i, (d_out, r) in enumerate(zip(outs, ranks)):
        G = torch.randn(n_rows, d_out, generator=g).to(torch.bfloat16)
        A = (torch.randn(d_in, r, generator=g) / math.sqrt(d_in)).to(torch.bfloat16)
        B = (torch.randn(r, d_out, generator=g) * 0.05).to(torch.bfloat16)
        ia = ib = None
        if (i, "A") not in frozen:
            ia = len(leaves)
            leaves.append(LeafOut(tuple(A.shape), torch.bfloat16))
            shapes.append(tuple(A.shape))
        if (i, "B") not in frozen:
            ib = len(leaves)
            leaves.append(LeafOut(tuple(B.shape), torch.bfloat16))
            shapes.append(tuple(B.shape))
        sites.append((G, A, B, ia, ib))
    return X, sites, leaves, shapes


def _plan(X, sites, leaves, shapes, seg, fuse, C=1.0, scaling=2.0):
    _, rnd = leaf_guards(shapes, [torch.bfloat16] * len(shapes))
    rel, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[C], effective=C, normalize_by=1.0,
                    guards=[(rel, ab, torch.bfloat16)])
    xd = X.to(DEV)
    lsites = [LoraSite(xd, G.to(DEV), A.to(DEV), B.to(DEV), scaling, a_leaf=ia, b_leaf=ib)
              for G, A, B, ia, ib in sites]
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=lsites, device=DEV,
                     fuse_g_side=fuse)
    res = plan.run()
    torch.cuda.synchronize()
    return plan, res


CASES = [
    # n_ex, T, lengths, d_in, d_outs, ranks, frozen
    (5, 96, [96, 33, 1, 70, 64], 136, [264], [8], ()),            # last chunk partial, length 1
    (3, 1081, [1081, 0, 517], 64, [512], [16], ()),               # longest segment, empty segment
    (4, 40, [40, 39, 17, 25], 96, [1000, 200], [12, 4], ()),      # ranks below 16, two sites share X
    (3, 64, [64, 50, 9], 128, [256, 136], [8, 8], ((0, "B"), (1, "A"))),  # frozen factors
    (4, 80, [80, 33, 1, 64], 520, [136], [16], ()),               # mirrored: d_in > d_out
    (3, 64, [64, 0, 40], 392, [128], [8], ((0, "B"),)),           # mirrored, frozen B
    (3, 1081, [1081, 5, 300], 264, [64], [16], ()),               # mirrored, longest segment
]


@pytest.mark.parametrize("n_ex,T,lengths,d_in,d_outs,ranks,frozen", CASES)
def test_fused_g_side_equals_two_pass(n_ex, T, lengths, d_in, d_outs, ranks, frozen):
    print(f"fused G side: n_ex={n_ex} T={T} d_in={d_in} d_outs={d_outs} ranks={ranks}", flush=True)
    seg = Segments.padded(n_ex, T, lengths)
    X, sites, leaves, shapes = _sites(n_ex * T, d_in, d_outs, ranks, frozen)
    p1, r1 = _plan(X, sites, leaves, shapes, seg, fuse=True)
    assert any(t[0] == "factor_project" and t[5] > 0 for t in p1.tables)
    p0, r0 = _plan(X, sites, leaves, shapes, seg, fuse=False)
    assert not any(t[0] == "factor_project" and t[5] > 0 for t in p0.tables)
    for a, b in zip(p1.pe_views(), p0.pe_views()):
        assert torch.equal(a, b)
    assert torch.equal(r1.norms, r0.norms)
    for a, b in zip(r1.leaves, r0.leaves):
        assert torch.equal(a, b)


@pytest.mark.parametrize("d_in,d_out", [(72, 328), (520, 72)])
def test_fused_g_side_unaligned_segments_match_oracle(d_in, d_out):
    # Packed rows: segment starts are not multiples of 8.
    print(f"fused, unaligned segments: d_in={d_in} d_out={d_out}", flush=True)
    lengths = [13, 37, 77, 0, 100]
    starts = [0, 13, 50, 127, 127]
    n_rows = 240
    seg = Segments(starts, lengths, list(range(5)), 5, n_rows)
    X, sites, leaves, shapes = _sites(n_rows, d_in, [d_out], [16], seed=5)
    p1, r1 = _plan(X, sites, leaves, shapes, seg, fuse=True, C=1e30)
    p0, r0 = _plan(X, sites, leaves, shapes, seg, fuse=False, C=1e30)
    assert torch.equal(r1.norms, r0.norms)
    G, A, B, _, _ = sites[0]
    dA, dB = lora_ref.lora_per_example(X, G, A, B, 2.0, starts, lengths)
    want = (dA.pow(2).sum((1, 2)) + dB.pow(2).sum((1, 2))).sqrt()
    got = r1.norms.double().cpu()
    assert torch.allclose(got, want, rtol=2e-2, atol=1e-30), (got, want)
    gb = r1.leaves[1].double().cpu()
    assert (gb - dB.sum(0)).norm() <= 2e-2 * dB.sum(0).norm()
    ga = r1.leaves[0].double().cpu()
    assert (ga - dA.sum(0)).norm() <= 2e-2 * dA.sum(0).norm()


@pytest.mark.parametrize("d_in,d_out", [(96, 200), (328, 72)])
def test_segment_past_the_fused_limit_takes_the_two_pass_path(d_in, d_out):
    """A segment longer than odp_factor_project_max_len() rows: the plan
    leaves the fused kernel out for that site even with fusion on, and the
    two-kernel path it takes instead matches the oracle."""
    limit = int(N.load().odp_factor_project_max_len())
    lengths = [limit + 37, 11, 0]
    T = limit + 37
    print(f"past the fused limit: limit={limit} lengths={lengths} d_in={d_in} d_out={d_out}", flush=True)
    seg = Segments.padded(3, T, lengths)
    X, sites, leaves, shapes = _sites(3 * T, d_in, [d_out], [16], seed=11)
    p1, r1 = _plan(X, sites, leaves, shapes, seg, fuse=True, C=1e30)
    assert not any(t[0] == "factor_project" and t[5] > 0 for t in p1.tables)
    G, A, B, _, _ = sites[0]
    starts = [i * T for i in range(3)]
    dA, dB = lora_ref.lora_per_example(X, G, A, B, 2.0, starts, lengths)
    want = (dA.pow(2).sum((1, 2)) + dB.pow(2).sum((1, 2))).sqrt()
    got = r1.norms.double().cpu()
    assert torch.allclose(got, want, rtol=2e-2, atol=1e-30), (got, want)
    ga, gb = r1.leaves[0].double().cpu(), r1.leaves[1].double().cpu()
    assert (ga - dA.sum(0)).norm() <= 2e-2 * dA.sum(0).norm()
    assert (gb - dB.sum(0)).norm() <= 2e-2 * dB.sum(0).norm()


@pytest.mark.parametrize("fuse", [True, False])
@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[4]])
def test_norms_square_the_stored_values(case, fuse):
    """The reference squares each per-example gradient as stored in the
    parameter dtype (clipping/_pytree.py:224-265 squares the bf16 leaf).  The
    kernels' squared norms must therefore be the fp32 squares of the bf16
    values they store, summed in fp64: equal to the sum over pe_views up to
    the fp64 summation order (rel 1e-12).  Squaring the unrounded fp32
    values instead differs by about 2^-9 / sqrt(n) relative, 1e-5 here."""
    n_ex, T, lengths, d_in, d_outs, ranks, frozen = case
    print(f"norms of stored values: fuse={fuse} d_in={d_in} d_outs={d_outs}", flush=True)
    seg = Segments.padded(n_ex, T, lengths)
    X, sites, leaves, shapes = _sites(n_ex * T, d_in, d_outs, ranks, frozen, seed=3)
    plan, res = _plan(X, sites, leaves, shapes, seg, fuse=fuse, C=1e30)
    want = torch.zeros(n_ex, dtype=torch.float64)
    for pe, lf in zip(plan.pe_views(), leaves):
        per = pe.view(n_ex, -1).float()  # one segment per example, in order
        assert pe.dtype == torch.bfloat16
        want += per.square().double().sum(1).cpu()
    got = res.norms.double().cpu().square()
    assert torch.allclose(got, want, rtol=1e-6, atol=0), (got, want)  # the stored norm is fp32
    # The fp32-rounded norm leaves 1e-7; the exact check runs on the fp64 partials.
    part = plan.part.double().sum(1).cpu()
    assert torch.allclose(part, want, rtol=1e-12, atol=0), ((part / want) - 1).abs().max()
