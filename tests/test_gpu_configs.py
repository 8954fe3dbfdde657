"""Parity at the shapes of the benchmark configurations (one layer of each at full size).

C1: Linear(768, 768) + LoRA r8 (alpha 16), batch 32 x 128, fp32, C = 1, noise 1.
C2: one GPT-2-small layer (q, k, v, o 768->768, fc 768->3072, proj 3072->768), LoRA r8,
    batch 64 x 512, bf16, per-example scale LogNormal(0, 1) so some examples clip.
C3: one Llama-3-8B layer (q, k, v, o, gate, up, down), LoRA r16, batch 16 x 1024 ragged
    lengths in [256, 1024], bf16, AUTO-S.
C4: one full-weight Llama-3-8B layer (7 linears), batch 8 x 4096, bf16, PerGroup with 7
    thresholds; stored, GEMM and token-Gram paths.
C5: one Mixtral-shaped MoE block, 8 experts with LoRA r16 on gate/up/down, batch 16 x 2048,
    top-2 routing, bf16.

The oracle forms the per-example gradients in fp64 on the CPU (oracle.lora_ref), applies
the reference clip / AUTO-S arithmetic per example and sums.  At C4 and C5 sizes the
per-example gradients (1.4e13 flops per C4 layer) are formed by plain fp32 torch.matmul on
the device instead, itself checked against the fp64 CPU oracle on a subset.  Tolerances:
fp32 rel 1e-5, bf16 rel 2e-2; masks compared away from the threshold band.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from opaque_amd import _native as N
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LinearSite, LoraSite, Segments
from opaque_amd.guard import guard_constants, leaf_guards
from opaque_amd.noise import add_noise_tree
from oracle import lora_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lora_sites(shapes, B, T, r, dtype, seed, lengths=None, g_scale=None, shared=None, products=False):
    """Sites of one layer; with ``products`` each also brings the seam's V = x A
    and U = g B^T (torch.matmul on the device in the site dtype, as the
    LoRA forward and its dx backward compute them)."""
    g = torch.Generator().manual_seed(seed)
    seg = Segments.padded(B, T, lengths)
    xs, sites, host = {}, [], []
    for li, (name, (d_in, d_out)) in enumerate(shapes.items()):
        key_ = (shared or {}).get(name, name)
        if key_ not in xs:
            xs[key_] = torch.randn(B * T, d_in, generator=g)
        x = xs[key_]
        gt = torch.randn(B * T, d_out, generator=g)
        if g_scale is not None:
            gt = gt * g_scale.repeat_interleave(T).view(-1, 1)
        for i, ln in enumerate(seg.lengths):
            gt[i * T + ln : (i + 1) * T] = 0.0  # padding rows carry no gradient
        A = torch.randn(d_in, r, generator=g) / math.sqrt(d_in)
        Bm = torch.randn(r, d_out, generator=g) * 0.02
        x, gt, A, Bm = (t.to(dtype) for t in (x, gt, A, Bm))
        xd, gd, Ad, Bd = x.to(DEV), gt.to(DEV), A.to(DEV), Bm.to(DEV)
        v = torch.matmul(xd, Ad) if products else None
        u = torch.matmul(gd, Bd.t()) if products else None
        sites.append(LoraSite(xd, gd, Ad, Bd, 2.0, a_leaf=2 * li, b_leaf=2 * li + 1, v=v, u=u))
        host.append((x, gt, A, Bm))
    return seg, sites, host


def _oracle(seg, host, s=2.0):
    pe, sq = [], torch.zeros(seg.n_ex, dtype=torch.float64)
    for x, gt, A, Bm in host:
        dA, dB = lora_ref.lora_per_example(x, gt, A, Bm, s, seg.starts, seg.lengths)
        pe += [dA, dB]
        sq += dA.pow(2).sum((1, 2)) + dB.pow(2).sum((1, 2))
    return pe, sq.sqrt()


def _run(seg, sites, leaves, dtype, mode, C, normalize_by):
    """Builds and runs the plan; a plan over sites that bring V and U must
    read them (odp_pack_planes) and project nothing."""
    shapes = [lf.shape for lf in leaves]
    _, rnd = leaf_guards(shapes, [dtype] * len(shapes))
    rel, ab = guard_constants(dtype, rnd)
    clip = ClipSpec(mode=mode, thresholds=[C], effective=C, gamma=0.01, normalize_by=normalize_by,
                    guards=[(rel, ab, dtype)])
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=sites, device=DEV)
    if sites and all(s.v is not None for s in sites):
        live = {t[0] for t in plan.tables if t[5] > 0}
        assert "planes" in live and not live & {"project", "factor_project"}, live
    res = plan.run()
    torch.cuda.synchronize()
    return res


def _check_lora(seg, host, res, *, mode, C, normalize_by, tol, band):
    pe, norms = _oracle(seg, host)
    assert torch.allclose(res.norms.double().cpu(), norms, rtol=tol, atol=0)
    fac = torch.clamp(C / norms, max=1.0) if mode == N.CLIP_FIXED else C / (norms + 0.01)
    fac = torch.where(torch.isfinite(fac), fac, torch.zeros_like(fac))
    for k, p in enumerate(pe):
        want = (fac[:, None, None] * p).sum(0) / normalize_by  # dA [d_in, r], dB [r, d_out]
        got = res.leaves[k].double().cpu()
        assert (got - want).norm() <= tol * want.norm() + 1e-12, k
    far = ((norms - C).abs() / C) > band
    assert torch.equal(res.clipped_total.cpu().bool()[far], (norms.float() > C)[far])
    return norms


@pytest.mark.parametrize("products", [False, True])
def test_config_c1(products):
    shapes = {"lin": (768, 768)}
    seg, sites, host = _lora_sites(shapes, 32, 128, 8, torch.float32, seed=1, products=products)
    leaves = [LeafOut((768, 8), torch.float32), LeafOut((8, 768), torch.float32)]
    res = _run(seg, sites, leaves, torch.float32, N.CLIP_FIXED, 1.0, 32.0)
    _check_lora(seg, host, res, mode=N.CLIP_FIXED, C=1.0, normalize_by=32.0, tol=1e-5, band=1e-6)
    # Noise: sigma = noise multiplier x max_norm = 1 x (1 / 32).
    from opaque_amd.random import fold_in, key
    from oracle import philox_ref

    seed = fold_in(key(0), 0).seed  # the step-0 key of gaussian_noise(key=key(0))
    flat = res.flat[torch.float32]
    noisy = add_noise_tree({"f": flat}, 1.0 / 32.0, seed)["f"]
    z = ((noisy - flat) * 32.0).double().cpu().numpy()
    want = philox_ref.gaussian_noise(np.zeros(z.size), 1.0, seed=seed, flat_offset=0)
    assert np.abs(z - want).max() < 1e-3  # same stream; fp32 device transform vs fp64 oracle
    from scipy import stats

    n = z.size  # 5-sigma bounds of the sample mean and standard deviation
    assert abs(z.mean()) < 5.0 / math.sqrt(n) and abs(z.std() - 1.0) < 5.0 * math.sqrt(0.5 / n)
    assert stats.kstest(z, "norm").pvalue > 0.01


@pytest.mark.parametrize("products", [False, True])
def test_config_c2_layer(products):
    shapes = {"q": (768, 768), "k": (768, 768), "v": (768, 768), "o": (768, 768), "fc": (768, 3072), "proj": (3072, 768)}
    shared = {"k": "q", "v": "q"}
    B, T = 64, 512
    g_scale = torch.exp(torch.randn(B, generator=torch.Generator().manual_seed(7))) * 0.02
    seg, sites, host = _lora_sites(shapes, B, T, 8, torch.bfloat16, seed=2, g_scale=g_scale, shared=shared,
                                   products=products)
    _, norms0 = _oracle(seg, host)
    C = float(norms0.median())
    leaves = []
    for d_in, d_out in shapes.values():
        leaves += [LeafOut((d_in, 8), torch.bfloat16), LeafOut((8, d_out), torch.bfloat16)]
    res = _run(seg, sites, leaves, torch.bfloat16, N.CLIP_FIXED, C, float(B))
    norms = _check_lora(seg, host, res, mode=N.CLIP_FIXED, C=C, normalize_by=float(B), tol=2e-2, band=1e-3)
    assert 0 < int((norms > C).sum()) < B  # some examples clip, some do not


@pytest.mark.parametrize("products", [False, True])
def test_config_c3_layer(products):
    shapes = {"q": (4096, 4096), "k": (4096, 1024), "v": (4096, 1024), "o": (4096, 4096),
              "gate": (4096, 14336), "up": (4096, 14336), "down": (14336, 4096)}
    shared = {"k": "q", "v": "q", "up": "gate"}
    B, T = 16, 1024
    lengths = torch.randint(256, T + 1, (B,), generator=torch.Generator().manual_seed(0)).tolist()
    seg, sites, host = _lora_sites(shapes, B, T, 16, torch.bfloat16, seed=3, lengths=lengths, shared=shared,
                                   products=products)
    leaves = []
    for d_in, d_out in shapes.values():
        leaves += [LeafOut((d_in, 16), torch.bfloat16), LeafOut((16, d_out), torch.bfloat16)]
    res = _run(seg, sites, leaves, torch.bfloat16, N.CLIP_AUTOS, 1.0, float(B))
    _check_lora(seg, host, res, mode=N.CLIP_AUTOS, C=1.0, normalize_by=float(B), tol=2e-2, band=1e-3)


C4_SHAPES = {"q": (4096, 4096), "k": (4096, 1024), "v": (4096, 1024), "o": (4096, 4096),
             "gate": (4096, 14336), "up": (4096, 14336), "down": (14336, 4096)}
C4_SHARED = {"q": "qkv", "k": "qkv", "v": "qkv", "o": "o", "gate": "gu", "up": "gu", "down": "down"}


def _c4_layer(seed):
    """One Llama-3-8B layer at C4's workload: batch 8 x 4096 tokens, bf16,
    output gradients scaled per example so that some examples clip."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    B, T = 8, 4096
    spread = torch.logspace(-1.0, 1.0, B, device=DEV).repeat_interleave(T).view(-1, 1)
    xs, sites = {}, []
    for name, (d_in, d_out) in C4_SHAPES.items():
        key_ = C4_SHARED[name]
        if key_ not in xs:
            xs[key_] = torch.randn(B * T, d_in, device=DEV, generator=gen).to(torch.bfloat16)
        g = (torch.randn(B * T, d_out, device=DEV, generator=gen) * spread * 1e-3).to(torch.bfloat16)
        sites.append((name, xs[key_], g))
    return B, T, sites


def _c4_norms(B, T, sites):
    """Plain PyTorch fp32 on the device: per-example M_s = G_s^T X_s by
    torch.matmul and its Frobenius norm, [n_sites, B] float64."""
    norms = torch.zeros(len(sites), B, dtype=torch.float64)
    for k, (_, x, g) in enumerate(sites):
        for s in range(B):
            m = torch.matmul(g[s * T : (s + 1) * T].float().t(), x[s * T : (s + 1) * T].float())
            norms[k, s] = m.double().pow(2).sum().sqrt().item()
    return norms


def _c4_sums(B, T, sites, fac, squares=False):
    """The reference's clipped sum from per-example M_s: M_s rounded to bf16 as
    vmap(grad) stores it, each scale.to(bf16) * M_s rounded to bf16, fp32 sum,
    bf16, / 8.  With squares, also the second moment: each clipped term
    squared in bf16, summed the same way (_clipped_fun.py:675-683,777-782)."""
    sums, sums2 = [], []
    for k, (_, x, g) in enumerate(sites):
        acc = acc2 = None
        for s in range(B):
            m = torch.matmul(g[s * T : (s + 1) * T].float().t(), x[s * T : (s + 1) * T].float()).to(torch.bfloat16)
            y = fac[k, s].to(DEV) * m
            t = y.float()
            acc = t if acc is None else acc + t
            if squares:
                t2 = y.square().float()
                acc2 = t2 if acc2 is None else acc2 + t2
        sums.append((acc.to(torch.bfloat16) / 8.0).cpu())
        if squares:
            sums2.append((acc2.to(torch.bfloat16) / 8.0).cpu())
    return (sums, sums2) if squares else sums


@pytest.mark.parametrize("path", ["stored", "gemm", "gram_gate_down", "moments"])
def test_config_c4_layer(path):
    """C4 at its workload: one full Llama-3-8B layer (7 full-weight linears),
    batch 8 x 4096, PerGroup with 7 thresholds (one per linear type), on the
    stored path, the clipped-sum GEMM path, with gate/down forced to the
    token-Gram norms, and with second moments and nothing stored (the
    moments kernel).  Group norms rel 2e-3 and the clipped sums (and second
    moments) rel 2e-2 against a plain fp32 reference; one example of k also
    against the fp64 CPU oracle."""
    print(f"C4 layer: path={path}", flush=True)
    B, T, sites = _c4_layer(seed=44)
    shapes = [(g.shape[1], x.shape[1]) for _, x, g in sites]
    _, rnd = leaf_guards(shapes, [torch.bfloat16] * len(shapes))
    rel, ab = guard_constants(torch.bfloat16, rnd)
    # Thresholds: each group's median norm, so that half the examples clip.
    norms = _c4_norms(B, T, sites)
    C = [float(norms[k].median()) for k in range(len(sites))]
    forms = {"gate": N.FORM_GRAM, "down": N.FORM_GRAM} if path == "gram_gate_down" else {}
    lins = [LinearSite(x, g, k, forms.get(name)) for k, (name, x, g) in enumerate(sites)]
    leaves = [LeafOut(shp, torch.bfloat16, group=k) for k, shp in enumerate(shapes)]
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=C, effective=math.sqrt(sum(c * c for c in C)), normalize_by=8.0,
                    guards=[(rel, ab, torch.bfloat16)])
    plan = GhostPlan(segments=Segments.padded(B, T), leaves=leaves, clip=clip, linear_sites=lins, device=DEV,
                     linear_pe_bytes=None if path == "stored" else 0, second_moment=path == "moments")
    res = plan.run()
    torch.cuda.synchronize()
    kinds = {t[1] for t in plan.tables if t[0] == "lin_norm" and t[5] > 0 and t[1] != N.FORM_OUTER_GUARDED}
    # Stored: every site takes the outer form (it stores).  Without storage
    # the engine picks the Gram identity for gate/up/down at T = 4096 (and
    # gate/down are forced to it), on the 256-row-block kernel.
    assert kinds == ({N.FORM_OUTER} if path == "stored" else {N.FORM_OUTER, N.FORM_GRAM256}), kinds
    assert (plan.lin_pe.numel() > 0) == (path == "stored")
    from oracle import dp_ref

    fac = torch.stack([dp_ref.finalize(torch.tensor(C[k], dtype=torch.float64) / norms[k], torch.bfloat16, rnd, True)
                       for k in range(len(sites))]).to(torch.bfloat16)
    sums, sums2 = _c4_sums(B, T, sites, fac, squares=True) if path == "moments" else (_c4_sums(B, T, sites, fac),
                                                                                        None)
    if path == "moments":
        assert {t[0] for t in plan.tables if t[5] > 0} >= {"lin_moments"}
        assert not any(t[0] in ("lin_sum", "lin_prescale") and t[5] > 0 for t in plan.tables)
        for k in range(len(sites)):
            want, got = sums2[k].double(), res.second_moment[k].double().cpu()
            assert (got - want).norm() <= 2e-2 * want.norm(), (k, ((got - want).norm() / want.norm()).item())
    got_n = res.group_norms.double().cpu()
    assert torch.allclose(got_n, norms, rtol=2e-3), (got_n / norms - 1).abs().max()
    for k in range(len(sites)):
        far = ((norms[k] - C[k]).abs() / C[k]) > 1e-3
        assert torch.equal(res.clipped[k].cpu().bool()[far], (norms[k].float() > C[k])[far]), k
        want, got = sums[k].double(), res.leaves[k].double().cpu()
        assert (got - want).norm() <= 2e-2 * want.norm(), (k, ((got - want).norm() / want.norm()).item())
    assert 0 < int(res.clipped.sum()) < res.clipped.numel()
    # fp64 oracle on the CPU for one example of k (4096 x 1024 per-example gradient).
    _, x, g = sites[1]
    pe = lora_ref.linear_per_example(x[:T].cpu().float(), g[:T].cpu().float(), [0], [T])
    assert abs(got_n[1, 0].item() / pe.pow(2).sum().sqrt().item() - 1.0) < 2e-3


def test_config_c5_moe():
    """C5 at its configured batch: one Mixtral-shaped MoE block, 8 experts with
    LoRA r16 on gate/up (4096 -> 14336) and down (14336 -> 4096), batch 16 x
    2048, top-2 routing (65,536 (token, expert) rows in per-(example, expert)
    segments).  Norms and clipped sums against plain fp32 on the device
    (rel 2e-2); expert 0 against the fp64 CPU oracle."""
    print("C5 MoE block at batch 16", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(5)
    B, T, E, k, H, I, r = 16, 2048, 8, 2, 4096, 14336, 16
    top = torch.randn(B, T, E, device=DEV, generator=gen).topk(k, dim=-1).indices
    sites, host, leaves = [], [], []
    for e in range(E):
        hit = (top == e).any(-1)  # [B, T]
        lengths = hit.sum(1).tolist()
        starts = [0] + list(np.cumsum(lengths)[:-1])
        n_rows = int(sum(lengths))
        seg = Segments([int(s) for s in starts], lengths, list(range(B)), B, n_rows)
        for name, (d_in, d_out) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
            x = torch.randn(n_rows, d_in, device=DEV, generator=gen).to(torch.bfloat16)
            gt = (torch.randn(n_rows, d_out, device=DEV, generator=gen) * 1e-2).to(torch.bfloat16)
            A = (torch.randn(d_in, r, device=DEV, generator=gen) / math.sqrt(d_in)).to(torch.bfloat16)
            Bm = (torch.randn(r, d_out, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
            n0 = len(leaves)
            leaves += [LeafOut((d_in, r), torch.bfloat16), LeafOut((r, d_out), torch.bfloat16)]
            sites.append(LoraSite(x, gt, A, Bm, 2.0, a_leaf=n0, b_leaf=n0 + 1, segments=seg))
            host.append((seg, x, gt, A, Bm))
    # Plain fp32 per-example LoRA factor gradients on the device.
    sq = torch.zeros(B, dtype=torch.float64)
    pes = []
    for seg, x, gt, A, Bm in host:
        xf, gf, Af, Bf = x.float(), gt.float(), A.float(), Bm.float()
        dA = torch.stack([2.0 * xf[s : s + n].t() @ (gf[s : s + n] @ Bf.t()) for s, n in zip(seg.starts, seg.lengths)])
        dB = torch.stack([2.0 * (xf[s : s + n] @ Af).t() @ gf[s : s + n] for s, n in zip(seg.starts, seg.lengths)])
        pes += [(seg, dA), (seg, dB)]
        sq += (dA.double().pow(2).sum((1, 2)) + dB.double().pow(2).sum((1, 2))).cpu()
    norms = sq.sqrt()
    C = float(norms.median())
    res = _run(Segments.padded(B, 1), sites, leaves, torch.bfloat16, N.CLIP_FIXED, C, float(B))
    assert torch.allclose(res.norms.double().cpu(), norms, rtol=2e-2)
    fac = torch.clamp(C / norms, max=1.0).to(DEV)
    for j, (seg, p) in enumerate(pes):
        want = (fac[:, None, None] * p.double()).sum(0) / float(B)
        got = res.leaves[j].double()
        assert (got - want).norm() <= 2e-2 * want.norm(), j
    assert 0 < int(res.clipped_total.sum()) < B
    # fp64 oracle on the CPU for expert 0's three sites.
    for j in range(3):
        seg, x, gt, A, Bm = host[j]
        dA, dB = lora_ref.lora_per_example(x.cpu(), gt.cpu(), A.cpu(), Bm.cpu(), 2.0, seg.starts, seg.lengths)
        assert (pes[2 * j][1].double().cpu() - dA).norm() <= 1e-4 * dA.norm()
        assert (pes[2 * j + 1][1].double().cpu() - dB).norm() <= 1e-4 * dB.norm()
