"""A GhostPlan rebound to a new call's inputs equals a plan built for them.

The drop-in clipped_grad keeps its last plan and, when the next call has the
same structure (plan_key), points it at the new inputs (GhostPlan.rebind)
instead of building tables and buffers again.  Checked here bit for bit
against fresh plans, for LoRA seams, materialised leaves, full-weight sites
on both storage paths, MoE segments and second moments; the previous call's
outputs must stay untouched (outputs are new tensors, as in the reference).
"""

from __future__ import annotations

import math
import time

import pytest
import torch

from opaque_amd import _native as N
from opaque_amd import capture
from opaque_amd.clipping import auto_clipped_grad, clipped_grad
from opaque_amd.engine import (LORA_PTRS, ClipSpec, GhostPlan, LeafOut, LinearSite, LoraSite, MaterializedLeaf,
                               Segments, plan_key)
from opaque_amd.guard import guard_constants, leaf_guards

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, n_ex=4, T=64, gram=True, products=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    bf = torch.bfloat16
    x = torch.randn(n_ex * T, 256, device=DEV, generator=g).to(bf)
    lora = []
    for k, d_out in enumerate((128, 384)):
        gt = torch.randn(n_ex * T, d_out, device=DEV, generator=g).to(bf) * 0.1
        A = (torch.randn(256, 16, device=DEV, generator=g) / 16).to(bf)
        B = (torch.randn(16, d_out, device=DEV, generator=g) * 0.02).to(bf)
        # products: the seam's own V = x A and U = g B^T come with the site.
        v = torch.matmul(x, A) if products else None
        u = torch.matmul(gt, B.t()) if products else None
        lora.append(LoraSite(x, gt, A, B, 2.0, a_leaf=2 * k, b_leaf=2 * k + 1, v=v, u=u))
    xl = torch.randn(n_ex * T, 136, device=DEV, generator=g).to(bf)
    lins = [LinearSite(xl, (torch.randn(n_ex * T, 72, device=DEV, generator=g) * 0.05).to(bf), 4),
            LinearSite(xl, (torch.randn(n_ex * T, 40, device=DEV, generator=g) * 0.05).to(bf), 5,
                       N.FORM_GRAM if gram else None)]
    mats = [MaterializedLeaf(torch.randn(n_ex, 33, device=DEV, generator=g), 6)]
    return lora, lins, mats


def _spec(thr):
    shapes = [(256, 16), (16, 128), (256, 16), (16, 384), (72, 136), (40, 136), (33,)]
    dts = [torch.bfloat16] * 6 + [torch.float32]
    _, rnd = leaf_guards(shapes, dts)
    guards = [(*guard_constants(torch.bfloat16, rnd), torch.bfloat16), (*guard_constants(torch.float32, rnd),
                                                                         torch.float32)]
    leaves = [LeafOut(s, torch.bfloat16 if i < 6 else torch.float32, group=i % 2, cls=0 if i < 6 else 1)
              for i, s in enumerate(shapes)]
    return leaves, ClipSpec(mode=N.CLIP_FIXED, thresholds=thr, effective=math.sqrt(sum(t * t for t in thr)),
                            normalize_by=4.0, guards=guards)


def _snapshot(res):
    return [t.clone() for t in res.leaves] + [res.norms.clone(), res.group_norms.clone(), res.scales.clone(),
                                              res.clipped.clone()] + [t.clone() for t in (res.second_moment or [])]


def _same(a, b):
    assert len(a) == len(b)
    for i, (u, v) in enumerate(zip(a, b)):
        assert torch.equal(u, v), i


def test_full_weight_second_moment_without_storage():
    """Second moments of full weights whose per-example gradients are not
    stored (linear_pe_bytes=0): the moments kernel forms each example's tile
    of M_s, rounds it to bf16 as the outer-norm kernel stores it and sums
    c_s m and bf16((c_s m)^2) per segment in order, so it must equal the
    stored path (outer norm with the bf16 store, then the scale-sum) bit for
    bit: first and second moments, norms and scales.  One example holds a
    NaN activation and another a pair of finite values whose product
    overflows float32; the reference zeroes both by nan_to_num
    (clipping/_pytree.py:520-527); one segment is empty."""
    print("rebind: second moment without stored full-weight gradients", flush=True)
    leaves, clip = _spec([0.5, 0.8])
    seg = Segments.padded(4, 64, [64, 0, 33, 64])
    l1, n1, m1 = _inputs(1, gram=False)
    xl, g0 = n1[0].x.clone(), n1[0].g.clone()
    xl[5, 17] = float("nan")  # example 0
    # Example 2, row 131: one entry of M_s is 1e40 (inf in float32); the
    # rest of the row's products stay small enough to square.
    xl[131] *= 1e-3
    g0[131] *= 1e-3
    xl[131, 40], g0[131, 9] = 1e20, 1e20
    n1 = [LinearSite(xl, g0, 4, N.FORM_OUTER), LinearSite(xl, n1[1].g, 5, N.FORM_OUTER)]
    kw = dict(clip=clip, lora_sites=l1, linear_sites=n1, materialized=m1, segments=seg, leaves=leaves,
              device=DEV, second_moment=True)
    stored = GhostPlan(linear_pe_bytes=None, **kw)
    assert stored.lin_pe.numel() > 0
    want = _snapshot(stored.run())
    plan = GhostPlan(linear_pe_bytes=0, **kw)
    assert plan.lin_pe.numel() == 0
    assert any(t[0] == "lin_moments" and t[5] > 0 for t in plan.tables)
    assert not any(t[0] in ("lin_sum", "lin_prescale") and t[5] > 0 for t in plan.tables)
    got = plan.run()
    torch.cuda.synchronize()
    _same(_snapshot(got), want)
    for k in (4, 5):
        assert torch.isfinite(got.leaves[k].float()).all() and torch.isfinite(got.second_moment[k].float()).all()
        assert got.second_moment[k].abs().sum() > 0


@pytest.mark.parametrize("products", [False, True])
@pytest.mark.parametrize("keyed", [False, True])
@pytest.mark.parametrize("pe_bytes,second_moment", [(None, False), (0, False), (None, True), (0, True)])
def test_rebind_equals_fresh_plan(pe_bytes, second_moment, keyed, products):
    print(f"rebind: pe_bytes={pe_bytes} second_moment={second_moment} keyed={keyed} products={products}",
          flush=True)
    leaves, clip1 = _spec([0.5, 0.8])
    _, clip2 = _spec([0.3, 1.1])  # thresholds change between calls (adaptive clipping)
    seg = Segments.padded(4, 64, [64, 10, 33, 64])
    l1, n1, m1 = _inputs(1, gram=not second_moment, products=products)
    l2, n2, m2 = _inputs(2, gram=not second_moment, products=products)
    kw = dict(segments=seg, leaves=leaves, device=DEV, second_moment=second_moment, linear_pe_bytes=pe_bytes)
    plan = GhostPlan(clip=clip1, lora_sites=l1, linear_sites=n1, materialized=m1, **kw)
    r1 = plan.run()
    first = _snapshot(r1)
    held = [t for t in r1.leaves]  # the tensors the first call handed out
    ptrs = torch.empty(LORA_PTRS * len(l2), dtype=torch.int64)
    k2 = plan_key(clip=clip2, lora_sites=l2, linear_sites=n2, materialized=m2, lora_ptrs=ptrs, **kw)
    assert plan.key == plan_key(clip=clip1, lora_sites=l1, linear_sites=n1, materialized=m1, **kw) == k2
    # keyed: the fast path when the host helper is built (addresses from plan_key)
    assert plan.rebind(l2, m2, n2, clip2, key=k2 if keyed else None, lora_ptrs=ptrs if keyed else None)
    r2 = plan.run()
    fresh = GhostPlan(clip=clip2, lora_sites=l2, linear_sites=n2, materialized=m2, **kw).run()
    torch.cuda.synchronize()
    _same(_snapshot(r2), _snapshot(fresh))
    _same([t for t in held], first[: len(held)])  # untouched by the second run
    assert not torch.equal(r2.leaves[0], first[0])
    # and back to the first inputs
    assert plan.rebind(l1, m1, n1, clip1)
    r3 = plan.run()
    torch.cuda.synchronize()
    _same(_snapshot(r3), first)


def test_rebind_refuses_a_different_layout():
    leaves, clip = _spec([0.5, 0.8])
    seg = Segments.padded(4, 64, [64, 10, 33, 64])
    l1, n1, m1 = _inputs(1)
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=l1, linear_sites=n1, materialized=m1,
                     device=DEV)
    l2, n2, m2 = _inputs(2)
    # q/k used to share their activation; now they do not.
    l2[1] = LoraSite(l2[1].x.clone(), l2[1].g, l2[1].A, l2[1].B, 2.0, a_leaf=2, b_leaf=3)
    assert not plan.rebind(l2, m2, n2, clip)
    k2 = plan_key(segments=seg, leaves=leaves, clip=clip, lora_sites=l2, linear_sites=n2, materialized=m2,
                  device=DEV)
    assert k2 != plan.key
    assert not plan.rebind(l2, m2, n2, clip, key=k2)
    # a transposed (same shape, other strides) output gradient changes the key
    l3, n3, m3 = _inputs(3)
    g_t = l3[0].g.t().contiguous().t()
    l3[0] = LoraSite(l3[0].x, g_t, l3[0].A, l3[0].B, 2.0, a_leaf=0, b_leaf=1)
    k3 = plan_key(segments=seg, leaves=leaves, clip=clip, lora_sites=l3, linear_sites=n3, materialized=m3,
                  device=DEV)
    assert k3 != plan.key


def _lora_loss(p, x, y):
    h = capture.lora_linear(x, p["W"], p["A1"], p["B1"], 2.0)
    h = torch.nn.functional.gelu(h)
    out = capture.lora_linear(h, p["W2"], p["A2"], p["B2"], 2.0)
    return ((out.float() - y.float()) ** 2).mean()


def test_drop_in_reuses_its_plan():
    """Two calls with the same structure: the second rebinds the first's
    plan, gives the result a fresh engine gives, is much cheaper on the
    host, and leaves the first call's outputs as they were."""
    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16
    d, h, r, n, T = 128, 256, 8, 8, 32
    p = {"W": (torch.randn(h, d, generator=g) / d**0.5).to(bf), "A1": (torch.randn(d, r, generator=g) / d**0.5).to(bf),
         "B1": (torch.randn(r, h, generator=g) * 0.02).to(bf), "W2": (torch.randn(d, h, generator=g) / h**0.5).to(bf),
         "A2": (torch.randn(h, r, generator=g) / h**0.5).to(bf), "B2": (torch.randn(r, d, generator=g) * 0.02).to(bf)}
    p = {k: v.to(DEV) for k, v in p.items()}
    frozen = {k: v for k, v in p.items() if k.startswith("W")}
    trainable = {k: v for k, v in p.items() if not k.startswith("W")}

    def loss(tr, x, y):
        return _lora_loss({**frozen, **tr}, x, y)

    batches = [(torch.randn(n, T, d, generator=g).to(bf).to(DEV), torch.randn(n, T, d, generator=g).to(bf).to(DEV))
               for _ in range(3)]
    fn, st = auto_clipped_grad(loss, R=0.5, normalize_by=float(n), batch_argnums=(1, 2), return_aux=True)
    (a, aux_a), _ = fn(trainable, *batches[0], state=st)
    plan0 = fn.engine._plan
    snap = {k: v.clone() for k, v in a.pytree.items()}
    norms_a = aux_a.grad_norms.clone()
    times = []
    for b in batches[1:]:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        (res, aux), _ = fn(trainable, *b, state=st)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
        assert fn.engine._plan is plan0  # rebound, not rebuilt
        fresh_fn, fst = auto_clipped_grad(loss, R=0.5, normalize_by=float(n), batch_argnums=(1, 2), return_aux=True)
        (want, waux), _ = fresh_fn(trainable, *b, state=fst)
        for k in want.pytree:
            assert torch.equal(res.pytree[k], want.pytree[k]), k
        assert torch.equal(aux.grad_norms, waux.grad_norms)
    for k in snap:
        assert torch.equal(a.pytree[k], snap[k]), k
    assert torch.equal(aux_a.grad_norms, norms_a)
    print(f"drop-in calls after the first: {[round(t * 1e3, 2) for t in times]} ms", flush=True)
