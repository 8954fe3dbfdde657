"""GPU parity of the full-weight linear kernels (outer / Gram norms, clipped-sum GEMM).

Per-example weight gradients M_i = G_i^T X_i are formed in fp64 on the CPU
by the oracle; the device never materialises them.  bf16 inputs, tolerance
rel 2e-2 against the oracle (the two device norm forms agree far closer).
"""

from __future__ import annotations

import pytest
import torch

from opaque_amd import _native as N
from opaque_amd import engine
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LinearSite, MaterializedLeaf, Segments, choose_form
from opaque_amd.guard import guard_constants, leaf_guards
from oracle import dp_ref, lora_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(n_ex, T, d_in, d_out, lengths, seed, scale_spread=True):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(n_ex * T, d_in, generator=g)
    G = torch.randn(n_ex * T, d_out, generator=g)
    if scale_spread:
        s = torch.logspace(-0.7, 0.7, n_ex).repeat_interleave(T).view(-1, 1)
        G = G * s
    seg = Segments.padded(n_ex, T, lengths)
    for i, ln in enumerate(seg.lengths):  # padding rows carry garbage that must be ignored
        X[i * T + ln : (i + 1) * T] = 1e4
        G[i * T + ln : (i + 1) * T] = -1e4
    return X.to(torch.bfloat16), G.to(torch.bfloat16), seg


def _plan(X, G, seg, *, C, mode, form, normalize_by=1.0, out_dtype=torch.bfloat16, pe_bytes=None):
    d_in, d_out = X.shape[1], G.shape[1]
    _, rnd = leaf_guards([(d_out, d_in)], [torch.bfloat16])
    rel, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=mode, thresholds=[C], effective=C, normalize_by=normalize_by,
                    guards=[(rel, ab, torch.bfloat16)])
    plan = GhostPlan(segments=seg, leaves=[LeafOut((d_out, d_in), out_dtype)], clip=clip,
                     linear_sites=[LinearSite(X.to(DEV), G.to(DEV), 0, form)], device=DEV,
                     linear_pe_bytes=pe_bytes)
    res = plan.run()
    torch.cuda.synchronize()
    return plan, res, rnd


def _ref_norms(X, G, seg):
    pe = lora_ref.linear_per_example(X.float(), G.float(), seg.starts, seg.lengths)
    return pe, pe.pow(2).sum((1, 2)).sqrt()


SHAPES = [
    # n_ex, T, d_in, d_out, lengths
    (4, 64, 128, 128, None),
    (5, 160, 200, 72, [160, 37, 0, 129, 64]),
    (3, 300, 136, 264, [300, 1, 255]),
    (2, 512, 384, 256, [512, 400]),
]


@pytest.mark.parametrize("n_ex,T,d_in,d_out,lengths", SHAPES)
@pytest.mark.parametrize("form", [N.FORM_OUTER, N.FORM_GRAM, N.FORM_GRAM256])
def test_linear_norms_match_oracle(n_ex, T, d_in, d_out, lengths, form):
    X, G, seg = _case(n_ex, T, d_in, d_out, lengths, seed=d_in + d_out)
    _, want = _ref_norms(X, G, seg)
    _, res, _ = _plan(X, G, seg, C=1e30, mode=N.CLIP_FIXED, form=form)
    got = res.norms.double().cpu()
    assert torch.allclose(got, want.float().double(), rtol=2e-3, atol=1e-6), (got, want)


# The 256-row-block Gram kernel: ragged segments across block edges, a
# one-row and an empty segment, n_seg >= 8 (work decoded in XCD order), up
# to five blocks (diagonal and off-diagonal pairs).
GRAM256_CASES = [
    # n_ex, T, d_in, d_out, lengths
    (3, 600, 136, 264, [600, 1, 300]),
    (9, 520, 128, 96, [520, 256, 255, 257, 0, 512, 100, 511, 3]),
    (2, 1100, 392, 200, [1100, 700]),
]


@pytest.mark.parametrize("n_ex,T,d_in,d_out,lengths", GRAM256_CASES)
def test_gram256_matches_oracle_and_gram128(n_ex, T, d_in, d_out, lengths, monkeypatch):
    """Norms of the 256-row-block kernel against the fp64 oracle (rel 2e-3)
    and against the 128-row-block kernel (rel 1e-5: the same products, fp32
    Gram blocks summed in fp64 in another order)."""
    print(f"gram256: n_ex={n_ex} T={T} d_in={d_in} d_out={d_out}", flush=True)
    X, G, seg = _case(n_ex, T, d_in, d_out, lengths, seed=T + d_in)
    _, want = _ref_norms(X, G, seg)
    plan, res, _ = _plan(X, G, seg, C=1e30, mode=N.CLIP_FIXED, form=N.FORM_GRAM)
    assert {t[1] for t in plan.tables if t[0] == "lin_norm" and t[5] > 0 and t[1] != N.FORM_OUTER_GUARDED} == {N.FORM_GRAM256}
    got = res.norms.double().cpu().clone()
    assert torch.allclose(got, want.float().double(), rtol=2e-3, atol=1e-6), (got, want)
    monkeypatch.setattr(engine, "GRAM256_MIN_LEN", 1 << 30)
    plan2, r2, _ = _plan(X, G, seg, C=1e30, mode=N.CLIP_FIXED, form=N.FORM_GRAM)
    assert {t[1] for t in plan2.tables if t[0] == "lin_norm" and t[5] > 0 and t[1] != N.FORM_OUTER_GUARDED} == {N.FORM_GRAM}
    assert torch.allclose(got, r2.norms.double().cpu(), rtol=1e-5, atol=1e-9)


def test_outer_and_gram_forms_agree():
    X, G, seg = _case(3, 256, 256, 192, [256, 100, 17], seed=9)
    _, r_outer, _ = _plan(X, G, seg, C=1e30, mode=N.CLIP_FIXED, form=N.FORM_OUTER)
    a = r_outer.norms.double().cpu().clone()
    _, r_gram, _ = _plan(X, G, seg, C=1e30, mode=N.CLIP_FIXED, form=N.FORM_GRAM)
    b = r_gram.norms.double().cpu()
    assert torch.allclose(a, b, rtol=1e-5), (a, b)


@pytest.mark.parametrize("mode", [N.CLIP_FIXED, N.CLIP_AUTOS])
@pytest.mark.parametrize("form,pe_bytes", [(N.FORM_OUTER, None), (N.FORM_OUTER, 0), (N.FORM_GRAM, None)])
def test_linear_clipped_sum_matches_oracle(mode, form, pe_bytes):
    """pe_bytes None: the outer form keeps each M_s (bf16) for odp_scale_sum; 0: the clipped-sum GEMM."""
    n_ex, T, d_in, d_out = 6, 96, 264, 136
    lengths = [96, 50, 7, 96, 0, 81]
    X, G, seg = _case(n_ex, T, d_in, d_out, lengths, seed=4)
    pe, norms = _ref_norms(X, G, seg)
    C = float(norms[norms > 0].median())
    plan, res, rnd = _plan(X, G, seg, C=C, mode=mode, form=form, normalize_by=6.0, pe_bytes=pe_bytes)
    assert plan.lin_pe.numel() == (n_ex * d_in * d_out if form == N.FORM_OUTER and pe_bytes is None else 0)
    # Oracle: reference clip_pytree per example (the per-example gradient rounded
    # to the bf16 parameter dtype, as vmap(grad) produces it), fp32 sum, cast, /6.
    outs = []
    for i in range(n_ex):
        leaf = {"w": pe[i].to(torch.bfloat16)}
        if mode == N.CLIP_FIXED:
            c, _, _ = dp_ref.clip_pytree(leaf, C)
        else:
            c, _, _ = dp_ref.auto_scale_pytree(leaf, C, 0.01)
        outs.append(c["w"])
    want = (torch.stack(outs).sum(0, dtype=torch.float32).to(torch.bfloat16) / 6.0).double()
    got = res.leaves[0].double().cpu()
    assert (got - want).norm() <= 2e-2 * want.norm()
    band = 1e-3
    far = ((norms - C).abs() / C) > band
    assert torch.equal(res.clipped_total.cpu().bool()[far], (norms.float() > C)[far])


def test_linear_with_materialized_leaf_per_group():
    """A linear weight and a materialised bias leaf in two clip groups."""
    n_ex, T, d_in, d_out = 4, 64, 128, 64
    X, G, seg = _case(n_ex, T, d_in, d_out, [64, 30, 64, 12], seed=2)
    pe, _ = _ref_norms(X, G, seg)
    bias_pe = torch.stack([G[s : s + ln].float().sum(0) for s, ln in zip(seg.starts, seg.lengths)])
    shapes = [(d_out, d_in), (d_out,)]
    _, rnd = leaf_guards(shapes, [torch.bfloat16, torch.float32])
    g_w, g_b = 0.5, 0.25
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[g_w, g_b], effective=(g_w**2 + g_b**2) ** 0.5,
                    guards=[(*guard_constants(torch.bfloat16, rnd), torch.bfloat16),
                            (*guard_constants(torch.float32, rnd), torch.float32)])
    plan = GhostPlan(segments=seg,
                     leaves=[LeafOut((d_out, d_in), torch.float32, group=0, cls=0),
                             LeafOut((d_out,), torch.float32, group=1, cls=1)],
                     clip=clip, linear_sites=[LinearSite(X.to(DEV), G.to(DEV), 0)],
                     materialized=[MaterializedLeaf(bias_pe.to(DEV), 1)], device=DEV)
    res = plan.run()
    torch.cuda.synchronize()

    class _PG:
        groups = {("w",): "w", ("b",): "b"}
        values = {"w": g_w, "b": g_b}

    outs_w, outs_b = [], []
    for i in range(n_ex):
        c, _, gn = dp_ref.clip_pytree({"w": pe[i].to(torch.bfloat16), "b": bias_pe[i]}, _PG)
        outs_w.append(c["w"].float())
        outs_b.append(c["b"])
    want_w = torch.stack(outs_w).sum(0).double()
    want_b = torch.stack(outs_b).sum(0).double()
    assert (res.leaves[0].double().cpu() - want_w).norm() <= 2e-2 * want_w.norm()
    assert (res.leaves[1].double().cpu() - want_b).norm() <= 1e-5 * want_b.norm()


# ---------------------------------------------------------------------------
# MoE: per-(example, expert) segments, each expert with its own rows
# (virtual groups b * E + e of opaque-patches/.../kernels/_grouped_moe.py:255)
# ---------------------------------------------------------------------------


def _moe_case(n_ex, T, E, k, d, h, r, dtype, seed):
    from opaque_amd.engine import LoraSite

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n_ex, T, d, generator=g)
    logits = torch.randn(n_ex, T, E, generator=g)
    top = logits.topk(k, dim=-1).indices  # [n_ex, T, k]
    sites, oracle = [], []
    for e in range(E):
        rows, starts, lengths, exs = [], [], [], []
        for b in range(n_ex):
            tok = [t for t in range(T) if bool((top[b, t] == e).any())]
            if not tok and b % 2 == 0:
                continue  # examples without tokens for e may omit their segment ...
            starts.append(len(rows))
            lengths.append(len(tok))  # ... or keep an empty one
            exs.append(b)
            rows += [(b, t) for t in tok]
        xe = torch.stack([x[b, t] for b, t in rows]) if rows else torch.zeros(0, d)
        ge = torch.randn(len(rows), h, generator=g) * (1.0 + e)
        A = torch.randn(d, r, generator=g) / d**0.5
        B = torch.randn(r, h, generator=g) * 0.1
        seg = Segments(starts, lengths, exs, n_ex, len(rows))
        xe, ge, A, B = (t.to(dtype) for t in (xe, ge, A, B))
        sites.append(LoraSite(xe.to(DEV), ge.to(DEV), A.to(DEV), B.to(DEV), 2.0, a_leaf=2 * e, b_leaf=2 * e + 1,
                              segments=seg))
        dA, dB = lora_ref.lora_per_example(xe, ge, A, B, 2.0, seg.starts, seg.lengths)
        oracle.append((seg, dA, dB))
    return sites, oracle


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_moe_expert_segments(dtype, tol):
    n_ex, T, E, k, d, h, r = 6, 40, 4, 2, 64, 96, 16
    sites, oracle = _moe_case(n_ex, T, E, k, d, h, r, dtype, seed=7)
    # Oracle: per example, squared norms summed over every expert's two leaves.
    sq = torch.zeros(n_ex, dtype=torch.float64)
    for seg, dA, dB in oracle:
        for i, b in enumerate(seg.examples):
            sq[b] += dA[i].pow(2).sum() + dB[i].pow(2).sum()
    norms = sq.sqrt()
    C = float(norms.median())
    shapes = [(d, r), (r, h)] * E
    _, rnd = leaf_guards(shapes, [dtype] * len(shapes))
    rel_, ab = guard_constants(dtype, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[C], effective=C, normalize_by=3.0, guards=[(rel_, ab, dtype)])
    plan = GhostPlan(segments=Segments.padded(n_ex, 1), leaves=[LeafOut(s, dtype) for s in shapes], clip=clip,
                     lora_sites=sites, device=DEV)
    res = plan.run()
    torch.cuda.synchronize()
    got = res.norms.double().cpu()
    assert torch.allclose(got, norms, rtol=tol, atol=0), (got, norms)
    fac = torch.clamp(C / norms, max=1.0)
    for e, (seg, dA, dB) in enumerate(oracle):
        ex = torch.tensor(seg.examples, dtype=torch.long)
        wa = (fac[ex][:, None, None] * dA).sum(0) / 3.0
        wb = (fac[ex][:, None, None] * dB).sum(0) / 3.0
        ga, gb = res.leaves[2 * e].double().cpu(), res.leaves[2 * e + 1].double().cpu()
        assert (ga - wa).norm() <= tol * wa.norm(), e
        assert (gb - wb).norm() <= tol * wb.norm(), e


@pytest.mark.parametrize("budget", [1 << 30, 100_000])
def test_prescaled_clipped_sum_equals_in_register(budget):
    """X' = c_i x_t staged by odp_linear_prescale gives the in-register result bit for bit.

    Packed segments with gaps (rows in no segment hold garbage), three sites
    on one X in two clip groups, a second X; the small budget splits the
    sites into several prescale chunks and leaves the widest X' in registers.
    """
    print(f"prescale: budget={budget}", flush=True)
    g = torch.Generator().manual_seed(17)
    n_rows = 300
    starts, lengths = [3, 40, 41, 150, 151], [37, 0, 100, 1, 140]
    seg = Segments(starts, lengths, [0, 1, 2, 3, 4], 5, n_rows)
    X1 = torch.randn(n_rows, 136, generator=g)
    X2 = torch.randn(n_rows, 520, generator=g) * 3
    for X in (X1, X2):
        X[:3] = 1e4
        X[291:] = -1e4
    X1, X2 = X1.to(torch.bfloat16).to(DEV), X2.to(torch.bfloat16).to(DEV)
    outs = [(X1, 72, 0), (X1, 200, 1), (X1, 64, 0), (X2, 96, 1)]
    leaves, lins, shapes = [], [], []
    for i, (X, d_out, grp) in enumerate(outs):
        G = (torch.randn(n_rows, d_out, generator=g) * (i + 1)).to(torch.bfloat16).to(DEV)
        lins.append(LinearSite(X, G, i))
        leaves.append(LeafOut((d_out, X.shape[1]), torch.bfloat16, group=grp))
        shapes.append((d_out, X.shape[1]))
    _, rnd = leaf_guards(shapes, [torch.bfloat16] * 4)
    rel, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[3.0, 20.0], effective=20.0, normalize_by=3.0,
                    guards=[(rel, ab, torch.bfloat16)])
    res = {}
    for b in (budget, 0):
        plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, linear_sites=lins, device=DEV,
                         prescale_bytes=b, linear_pe_bytes=0)
        r = plan.run()
        torch.cuda.synchronize()
        res[b] = ([t.clone() for t in r.leaves], r.scales.clone(), plan)
    pre = [t for t in res[budget][2].tables if t[0] == "lin_prescale" and t[5] > 0]
    assert len(pre) == (1 if budget == 1 << 30 else 3)
    assert not any(t[0] == "lin_prescale" and t[5] > 0 for t in res[0][2].tables)
    assert torch.equal(res[budget][1], res[0][1])
    assert (res[0][1] < 1).any()  # some examples clip
    for a, b in zip(res[budget][0], res[0][0]):
        assert torch.equal(a, b)


def _multi_site(seed=23):
    g = torch.Generator().manual_seed(seed)
    n_rows = 200
    seg = Segments([0, 60, 61, 130], [60, 1, 69, 70], [0, 1, 2, 3], 4, n_rows)
    X = (torch.randn(n_rows, 136, generator=g)).to(torch.bfloat16).to(DEV)
    outs = [72, 264, 40, 128]
    leaves, lins, shapes = [], [], []
    for i, d_out in enumerate(outs):
        G = (torch.randn(n_rows, d_out, generator=g) * (0.5 + i)).to(torch.bfloat16).to(DEV)
        lins.append(LinearSite(X, G, i, N.FORM_OUTER))
        leaves.append(LeafOut((d_out, 136), torch.float32, group=i % 2))
        shapes.append((d_out, 136))
    _, rnd = leaf_guards(shapes, [torch.bfloat16] * 4)
    rel, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[4.0, 30.0], effective=30.0, normalize_by=2.0,
                    guards=[(rel, ab, torch.bfloat16)])
    return seg, leaves, lins, clip


def test_stored_linear_gradients_within_a_budget():
    """A budget that holds two of four sites' per-example gradients: those two are
    summed from storage, the other two by the GEMM; norms are identical either way."""
    print("stored linear gradients: partial budget", flush=True)
    seg, leaves, lins, clip = _multi_site()
    res = {}
    for name, b in (("all", None), ("none", 0), ("part", 4 * 136 * (72 + 264) * 2)):
        plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, linear_sites=lins, device=DEV,
                         linear_pe_bytes=b)
        r = plan.run()
        torch.cuda.synchronize()
        res[name] = ([t.clone() for t in r.leaves], r.norms.clone(), plan.lin_pe.numel())
    assert res["part"][2] == 4 * 136 * (72 + 264) and res["none"][2] == 0
    assert torch.equal(res["all"][1], res["none"][1]) and torch.equal(res["part"][1], res["none"][1])
    for k in range(4):
        ref = res["none"][0][k].double()
        for name in ("all", "part"):
            got = res[name][0][k].double()
            assert (got - ref).norm() <= 1e-2 * ref.norm(), (name, k)
    # Sites 0 and 1 of the partial plan come from storage, 2 and 3 from the GEMM.
    for k in (2, 3):
        assert torch.equal(res["part"][0][k], res["none"][0][k])
    for k in (0, 1):
        assert torch.equal(res["part"][0][k], res["all"][0][k])


@pytest.mark.parametrize("pe_bytes", [None, 0])
def test_linear_gradients_second_moment(pe_bytes):
    """Second moments of full weights, with the per-example gradients stored
    (scale-sum over storage) or not (the moments kernel): both against the
    oracle's per-example gradients, clipped and squared in bf16."""
    print(f"linear gradients: second moment, linear_pe_bytes={pe_bytes}", flush=True)
    seg, leaves, lins, clip = _multi_site(seed=29)
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, linear_sites=lins, device=DEV,
                     second_moment=True, linear_pe_bytes=pe_bytes)
    assert (plan.lin_pe.numel() > 0) == (pe_bytes is None)
    r = plan.run()
    torch.cuda.synchronize()
    scales = r.scales.cpu()
    for k, ls in enumerate(lins):
        X, G = ls.x.cpu(), ls.g.cpu()
        pe = lora_ref.linear_per_example(X.float(), G.float(), seg.starts, seg.lengths).to(torch.bfloat16)
        # clip_pytree's `scale.to(bf16) * leaf` and the square of the clipped
        # bf16 leaf, each rounded to bf16, summed in fp32, then / 2.
        c = scales[0, leaves[k].group].to(torch.bfloat16).view(-1, 1, 1)
        y = c * pe
        want = (y.sum(0, dtype=torch.float32) / 2.0).double()
        want2 = (y.square().sum(0, dtype=torch.float32) / 2.0).double()
        assert (r.leaves[k].double().cpu() - want).norm() <= 2e-4 * want.norm(), k
        assert (r.second_moment[k].double().cpu() - want2).norm() <= 2e-4 * want2.norm(), k


def test_storage_takes_the_outer_form():
    """Short examples favour the Gram form for the norms alone; with room to
    store the per-example gradients the outer form (which stores them) is
    taken instead, and both plans agree."""
    print("form choice with storage", flush=True)
    X, G, seg = _case(4, 64, 512, 512, [64, 40, 64, 9], seed=31)
    assert choose_form(64, 512, 512) == N.FORM_GRAM
    res = {}
    for b in (None, 0):
        plan, r, _ = _plan(X, G, seg, C=5.0, mode=N.CLIP_FIXED, form=None, pe_bytes=b)
        kinds = {t[1] for t in plan.tables if t[0] == "lin_norm" and t[5] > 0 and t[1] != N.FORM_OUTER_GUARDED}
        assert kinds == ({N.FORM_OUTER} if b is None else {N.FORM_GRAM}), (b, kinds)
        res[b] = (r.leaves[0].double().cpu(), r.norms.double().cpu())
    assert torch.allclose(res[None][1], res[0][1], rtol=1e-4)
    assert (res[None][0] - res[0][0]).norm() <= 1e-2 * res[0][0].norm()


# Paths a full-weight site can take: (norm form, linear_pe_bytes, prescale_bytes).
_PATHS = {
    "stored": (None, None, 8 << 30),        # outer norms store each M_s; clipped sum over storage
    "gemm_outer": (N.FORM_OUTER, 0, 8 << 30),  # outer norms; prescaled X' and the clipped-sum GEMM
    "gemm_gram": (N.FORM_GRAM, 0, 8 << 30),    # token-Gram norms; prescaled X' and the GEMM
    "gemm_inreg": (N.FORM_GRAM, 0, 0),      # token-Gram norms; clip factors applied in registers
    "gemm_gram256": (N.FORM_GRAM256, 0, 8 << 30),  # 256-row-block Gram norms; prescaled X' and the GEMM
}


@pytest.mark.parametrize("kind", ["clean", "nan_x", "inf_g", "both"])
@pytest.mark.parametrize("path", sorted(_PATHS))
def test_non_finite_entries_are_zeroed(path, kind):
    """Non-finite activations / output gradients make whole columns / rows of
    one example's weight gradient non-finite.  The reference zeroes the
    non-finite per-example entries before the norm and the scale
    (nan_to_num, clipping/_pytree.py:520-527) and its test asserts a finite
    clipped sum (test_clipped_grad.py:64-87); every path does the same and
    reports it through linear_finite().  Non-finite values in padding rows
    (in no segment) are ignored."""
    print(f"non-finite entries: path={path} kind={kind}", flush=True)
    form, pe_bytes, pre_bytes = _PATHS[path]
    n_ex, T, d_in, d_out = 4, 48, 136, 72
    X, G, seg = _case(n_ex, T, d_in, d_out, [48, 30, 48, 20], seed=41)
    X[T + 40, 3] = float("nan")  # example 1 has 30 rows: a padding row
    if kind in ("nan_x", "both"):
        X[T + 5, 17] = float("nan")  # example 1, feature 17
    if kind in ("inf_g", "both"):
        G[2 * T + 40, 3] = float("inf")  # example 2, output 3
        G[3 * T + 2, 70] = float("-inf")  # example 3, output 70
        X[3 * T + 7, 130] = float("inf")  # example 3, feature 130
    pe, _ = _ref_norms(X, G, seg)
    if kind == "nan_x":
        assert torch.isnan(pe[1][:, 17]).all() and torch.isfinite(pe[0]).all()
    finite = torch.nan_to_num(pe, nan=0.0, posinf=0.0, neginf=0.0)
    C = float(finite.pow(2).sum((1, 2)).sqrt().median())
    d_in, d_out = X.shape[1], G.shape[1]
    _, rnd = leaf_guards([(d_out, d_in)], [torch.bfloat16])
    rel_, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[C], effective=C, normalize_by=2.0,
                    guards=[(rel_, ab, torch.bfloat16)])
    plan = GhostPlan(segments=seg, leaves=[LeafOut((d_out, d_in), torch.bfloat16)], clip=clip,
                     linear_sites=[LinearSite(X.to(DEV), G.to(DEV), 0, form)], device=DEV,
                     linear_pe_bytes=pe_bytes, prescale_bytes=pre_bytes)
    res = plan.run()
    finite_flag = bool(plan.linear_finite().item())
    torch.cuda.synchronize()
    assert (plan.lin_pe.numel() > 0) == (path == "stored")
    kinds = {t[1] for t in plan.tables if t[0] == "lin_norm" and t[5] > 0 and t[1] != N.FORM_OUTER_GUARDED}
    assert kinds == {form if form in (N.FORM_GRAM, N.FORM_GRAM256) else N.FORM_OUTER}
    outs, norms = [], []
    for i in range(n_ex):
        c, nrm, _ = dp_ref.clip_pytree({"w": pe[i].to(torch.bfloat16)}, C)
        outs.append(c["w"])
        norms.append(nrm)
    want = (torch.stack(outs).sum(0, dtype=torch.float32).to(torch.bfloat16) / 2.0).double()
    got = res.leaves[0].double().cpu()
    assert torch.isfinite(got).all()
    assert (got - want).norm() <= 2e-2 * want.norm()
    assert torch.allclose(res.norms.double().cpu(), torch.stack(norms).double(), rtol=2e-3)
    assert finite_flag == (kind == "clean")
    if path != "stored":
        words = (d_in + 31) // 32
        xmask = plan.nf_mask[: n_ex * words].view(n_ex, words).cpu()
        want_cols = {"clean": [], "nan_x": [(1, 17)], "inf_g": [(3, 130)], "both": [(1, 17), (3, 130)]}[kind]
        got_cols = [(s, 32 * w + b) for s in range(n_ex) for w in range(words) for b in range(32)
                    if (int(xmask[s, w]) >> b) & 1]
        assert got_cols == want_cols


def _overflow_case(seed=41):
    """Four examples of 64 rows (one empty).  Example 1: one entry of M is
    1e40, past float32 (the reference zeroes it; the rest of the example
    stays small, so its norm is finite).  Example 3: one entry of M is 1e20,
    whose square overflows float32 (the reference's norm is inf, so its
    scale is 0).  Example 0 is ordinary."""
    g = torch.Generator().manual_seed(seed)
    n_ex, T, d_in, d_out = 4, 64, 192, 136
    X = torch.randn(n_ex * T, d_in, generator=g)
    G = torch.randn(n_ex * T, d_out, generator=g) * 0.1
    seg = Segments.padded(n_ex, T, [64, 50, 0, 64])
    for row, big in ((T + 7, 1e20), (3 * T + 11, 1e10)):
        X[row] *= 1e-3
        G[row] *= 1e-3
        X[row, 40], G[row, 9] = big, big
    return X.to(torch.bfloat16), G.to(torch.bfloat16), seg


@pytest.mark.parametrize("form", [N.FORM_GRAM, N.FORM_GRAM256, N.FORM_OUTER])
@pytest.mark.parametrize("mode", [N.CLIP_FIXED, N.CLIP_AUTOS])
def test_overflowing_segments_take_the_exact_forms(form, mode):
    """Without stored gradients the Gram norms and the clipped-sum GEMM
    would carry such products as huge finite values or inf; the segments at
    risk are routed to the outer-form norms and the moments kernel, which
    form M_s tile by tile.  Results match the stored path (which forms and
    stores every M_s): the same inf norm and zero contribution for example
    3, the same zeroed entry for example 1, all_finite false."""
    print(f"overflow routing: form={form} mode={mode}", flush=True)
    X, G, seg = _overflow_case()
    C = 0.5
    _, want, _ = _plan(X, G, seg, C=C, mode=mode, form=None, pe_bytes=None, out_dtype=torch.float32)
    plan, got, _ = _plan(X, G, seg, C=C, mode=mode, form=form, pe_bytes=0, out_dtype=torch.float32)
    assert plan.lin_pe.numel() == 0
    live = {(t[0], t[1]) for t in plan.tables if t[5] > 0}
    if form == N.FORM_OUTER:
        assert ("lin_moments", 1) in live  # the guarded fallback of the GEMM
    else:
        assert ("lin_norm", N.FORM_OUTER_GUARDED) in live
    wn, gn = want.norms.double().cpu(), got.norms.double().cpu()
    assert torch.isinf(wn[3]) and torch.isinf(gn[3]) and torch.isfinite(wn[:3]).all()
    assert torch.allclose(gn[:3], wn[:3], rtol=1e-5), (gn, wn)
    assert torch.equal(got.scales.cpu()[..., 3], torch.zeros_like(got.scales.cpu()[..., 3]))
    assert torch.equal(got.clipped_total.cpu(), want.clipped_total.cpu())
    a, b = got.leaves[0].double().cpu(), want.leaves[0].double().cpu()
    assert torch.isfinite(a).all()
    assert (a - b).norm() <= 1e-4 * b.norm(), ((a - b).norm() / b.norm()).item()
    assert not bool(plan.linear_finite())
    # The oracle on the CPU: per-example gradients in bf16 (inf where they
    # overflow), nan_to_num, the reference's clip.
    pe = lora_ref.linear_per_example(X.float(), G.float(), seg.starts, seg.lengths).float().to(torch.bfloat16)
    assert torch.isinf(pe[1].float()).any()
    ref, raux = dp_ref.clipped_grad(lambda p, m: (p * m.float()).sum(), torch.zeros(pe.shape[1:]), (pe,),
                                    clipping_norm=C, autos=mode == N.CLIP_AUTOS)
    assert torch.isinf(raux["norms"][3])
    assert torch.allclose(gn[:3], raux["norms"][:3].double(), rtol=2e-2), (gn, raux["norms"])
