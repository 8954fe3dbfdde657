"""Parity at the shapes of the benchmark configurations (one layer of each at full size).

C1: Linear(768, 768) + LoRA r8 (alpha 16), batch 32 x 128, fp32, C = 1, noise 1.
C2: one GPT-2-small layer (q, k, v, o 768->768, fc 768->3072, proj 3072->768), LoRA r8,
    batch 64 x 512, bf16, per-example scale LogNormal(0, 1) so some examples clip.
C3: one Llama-3-8B layer (q, k, v, o, gate, up, down), LoRA r16, batch 16 x 1024 ragged
    lengths in [256, 1024], bf16, AUTO-S.
C4: one full-weight k projection (4096 -> 1024), batch 2 x 4096, bf16, Gram and outer forms.
C5: one Mixtral-shaped MoE block, 8 experts with LoRA r16 on gate/up/down, batch 4 x 2048
    (of the configured 16), top-2 routing, bf16.

The oracle forms the per-example gradients in fp64 on the CPU (oracle.lora_ref), applies
the reference clip / AUTO-S arithmetic per example and sums.  Tolerances: fp32 rel 1e-5,
bf16 rel 2e-2; masks compared away from the threshold band.
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


def _lora_sites(shapes, B, T, r, dtype, seed, lengths=None, g_scale=None, shared=None):
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
        sites.append(LoraSite(x.to(DEV), gt.to(DEV), A.to(DEV), Bm.to(DEV), 2.0, a_leaf=2 * li, b_leaf=2 * li + 1))
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
    shapes = [lf.shape for lf in leaves]
    _, rnd = leaf_guards(shapes, [dtype] * len(shapes))
    rel, ab = guard_constants(dtype, rnd)
    clip = ClipSpec(mode=mode, thresholds=[C], effective=C, gamma=0.01, normalize_by=normalize_by,
                    guards=[(rel, ab, dtype)])
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=sites, device=DEV)
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


def test_config_c1():
    shapes = {"lin": (768, 768)}
    seg, sites, host = _lora_sites(shapes, 32, 128, 8, torch.float32, seed=1)
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


def test_config_c2_layer():
    shapes = {"q": (768, 768), "k": (768, 768), "v": (768, 768), "o": (768, 768), "fc": (768, 3072), "proj": (3072, 768)}
    shared = {"k": "q", "v": "q"}
    B, T = 64, 512
    g_scale = torch.exp(torch.randn(B, generator=torch.Generator().manual_seed(7))) * 0.02
    seg, sites, host = _lora_sites(shapes, B, T, 8, torch.bfloat16, seed=2, g_scale=g_scale, shared=shared)
    _, norms0 = _oracle(seg, host)
    C = float(norms0.median())
    leaves = []
    for d_in, d_out in shapes.values():
        leaves += [LeafOut((d_in, 8), torch.bfloat16), LeafOut((8, d_out), torch.bfloat16)]
    res = _run(seg, sites, leaves, torch.bfloat16, N.CLIP_FIXED, C, float(B))
    norms = _check_lora(seg, host, res, mode=N.CLIP_FIXED, C=C, normalize_by=float(B), tol=2e-2, band=1e-3)
    assert 0 < int((norms > C).sum()) < B  # some examples clip, some do not


def test_config_c3_layer():
    shapes = {"q": (4096, 4096), "k": (4096, 1024), "v": (4096, 1024), "o": (4096, 4096),
              "gate": (4096, 14336), "up": (4096, 14336), "down": (14336, 4096)}
    shared = {"k": "q", "v": "q", "up": "gate"}
    B, T = 16, 1024
    lengths = torch.randint(256, T + 1, (B,), generator=torch.Generator().manual_seed(0)).tolist()
    seg, sites, host = _lora_sites(shapes, B, T, 16, torch.bfloat16, seed=3, lengths=lengths, shared=shared)
    leaves = []
    for d_in, d_out in shapes.values():
        leaves += [LeafOut((d_in, 16), torch.bfloat16), LeafOut((16, d_out), torch.bfloat16)]
    res = _run(seg, sites, leaves, torch.bfloat16, N.CLIP_AUTOS, 1.0, float(B))
    _check_lora(seg, host, res, mode=N.CLIP_AUTOS, C=1.0, normalize_by=float(B), tol=2e-2, band=1e-3)


@pytest.mark.parametrize("form", [N.FORM_OUTER, N.FORM_GRAM])
def test_config_c4_linear(form):
    g = torch.Generator().manual_seed(4)
    B, T, d_in, d_out = 2, 4096, 4096, 1024
    X = torch.randn(B * T, d_in, generator=g).to(torch.bfloat16)
    G = torch.randn(B * T, d_out, generator=g).to(torch.bfloat16)
    seg = Segments.padded(B, T)
    pe = lora_ref.linear_per_example(X.float(), G.float(), seg.starts, seg.lengths)
    norms = pe.pow(2).sum((1, 2)).sqrt()
    C = float(norms.mean())
    _, rnd = leaf_guards([(d_out, d_in)], [torch.bfloat16])
    rel, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[C], effective=C, normalize_by=8.0,
                    guards=[(rel, ab, torch.bfloat16)])
    plan = GhostPlan(segments=seg, leaves=[LeafOut((d_out, d_in), torch.bfloat16)], clip=clip,
                     linear_sites=[LinearSite(X.to(DEV), G.to(DEV), 0, form)], device=DEV)
    res = plan.run()
    torch.cuda.synchronize()
    assert torch.allclose(res.norms.double().cpu(), norms, rtol=2e-3)
    fac = torch.clamp(C / norms, max=1.0)
    want = (fac[:, None, None] * pe).sum(0) / 8.0
    got = res.leaves[0].double().cpu()
    assert (got - want).norm() <= 2e-2 * want.norm()


def test_config_c5_moe():
    g = torch.Generator().manual_seed(5)
    B, T, E, k, H, I, r = 4, 2048, 8, 2, 4096, 14336, 16
    top = torch.randn(B, T, E, generator=g).topk(k, dim=-1).indices
    sites, host, leaves = [], [], []
    for e in range(E):
        rows, starts, lengths = [], [], []
        for b in range(B):
            tok = torch.nonzero((top[b] == e).any(-1)).view(-1).tolist()
            starts.append(len(rows))
            lengths.append(len(tok))
            rows += [b * T + t for t in tok]
        seg = Segments(starts, lengths, list(range(B)), B, len(rows))
        for name, (d_in, d_out) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
            x = torch.randn(len(rows), d_in, generator=g).to(torch.bfloat16)
            gt = torch.randn(len(rows), d_out, generator=g).to(torch.bfloat16)
            A = (torch.randn(d_in, r, generator=g) / math.sqrt(d_in)).to(torch.bfloat16)
            Bm = (torch.randn(r, d_out, generator=g) * 0.02).to(torch.bfloat16)
            n0 = len(leaves)
            leaves += [LeafOut((d_in, r), torch.bfloat16), LeafOut((r, d_out), torch.bfloat16)]
            sites.append(LoraSite(x.to(DEV), gt.to(DEV), A.to(DEV), Bm.to(DEV), 2.0, a_leaf=n0, b_leaf=n0 + 1,
                                  segments=seg))
            host.append((seg, x, gt, A, Bm))
    sq = torch.zeros(B, dtype=torch.float64)
    pes = []
    for seg, x, gt, A, Bm in host:
        dA, dB = lora_ref.lora_per_example(x, gt, A, Bm, 2.0, seg.starts, seg.lengths)
        pes += [(seg, dA), (seg, dB)]
        for i, b in enumerate(seg.examples):
            sq[b] += dA[i].pow(2).sum() + dB[i].pow(2).sum()
    norms = sq.sqrt()
    C = float(norms.median())
    res = _run(Segments.padded(B, 1), sites, leaves, torch.bfloat16, N.CLIP_FIXED, C, float(B))
    assert torch.allclose(res.norms.double().cpu(), norms, rtol=2e-2)
    fac = torch.clamp(C / norms, max=1.0)
    for k, (seg, p) in enumerate(pes):
        ex = torch.tensor(seg.examples, dtype=torch.long)
        want = (fac[ex][:, None, None] * p).sum(0) / float(B)
        got = res.leaves[k].double().cpu()
        assert (got - want).norm() <= 2e-2 * want.norm(), k
