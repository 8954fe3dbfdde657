"""GPU parity of the drop-in ``clipped_grad`` / ``auto_clipped_grad`` against the CPU oracle.

Both sides differentiate the same per-example loss; the oracle restates the
reference's vmap(grad) + clip_pytree + fp32 sum on the CPU, the product runs
the HIP kernels (seam capture for LoRA factors, materialised leaves for the
rest).  Tolerances: fp32 rel <= 1e-5, bf16 rel <= 2e-2 (global relative
error of each leaf and of the norms).
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import dp_ref
from opaque_amd import capture
from opaque_amd.clipping import (
    AutoClippedGradAux,
    ClippedGradAux,
    ClippingStats,
    auto_clipped_grad,
    clipped_grad,
    per_group,
)
from opaque_amd.types import ClippedPytree, PerGroup, SecondMomentClippingOutput

pytestmark = pytest.mark.gpu

DEV = "cuda"


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.norm().item()
    return (a - b).norm().item() / den if den > 0 else (a - b).norm().item()


def _plain_lora(x, W, A, B, s, bias=None):
    out = x @ W.t() + s * ((x @ A) @ B)
    return out if bias is None else out + bias


def _peft(op):
    def f(x, W, a_w, b_w, s, bias=None):
        if op is None:
            return _plain_lora(x, W, a_w.t(), b_w.t(), s, bias)
        return op(x, W, a_w, b_w, s, bias)

    return f


def make_model(dtype, d=32, h=64, r=8, seed=0, layers=2):
    """A small transformer-ish MLP stack: LoRA on in/out projections, trainable norm weights."""
    g = torch.Generator().manual_seed(seed)

    def rn(*s, scale=1.0):
        return (torch.randn(*s, generator=g) * scale).to(dtype)

    frozen, train = {}, {}
    for li in range(layers):
        frozen[f"l{li}.up.W"] = rn(h, d, scale=d**-0.5)
        frozen[f"l{li}.down.W"] = rn(d, h, scale=h**-0.5)
        train[f"l{li}.up.lora_A"] = rn(r, d, scale=d**-0.5)
        train[f"l{li}.up.lora_B"] = rn(h, r, scale=0.2)
        train[f"l{li}.down.lora_A"] = rn(r, h, scale=h**-0.5)
        train[f"l{li}.down.lora_B"] = rn(d, r, scale=0.2)
        train[f"l{li}.norm"] = (1.0 + 0.1 * torch.randn(d, generator=g)).to(dtype)
    return frozen, train


def model_loss(op, frozen, layers=2, s=2.0):
    lora = _peft(op)

    def loss(params, x, y):
        hcur = x
        for li in range(layers):
            z = hcur * params[f"l{li}.norm"]
            u = lora(z, frozen[f"l{li}.up.W"], params[f"l{li}.up.lora_A"], params[f"l{li}.up.lora_B"], s)
            u = torch.nn.functional.gelu(u)
            hcur = hcur + lora(u, frozen[f"l{li}.down.W"], params[f"l{li}.down.lora_A"],
                               params[f"l{li}.down.lora_B"], s)
        return ((hcur.float() - y.float()) ** 2).mean()

    return loss


def to(tree, dev):
    return {k: v.to(dev) for k, v in tree.items()}


def run_both(dtype, *, n=6, T=16, autos=False, C=None, normalize_by=1.0, second_moment=False,
             return_aux=True, microbatch=None, out_dtype=None, seed=0):
    frozen, train = make_model(dtype, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(n, T, 32, generator=g).to(dtype)
    y = torch.randn(n, T, 32, generator=g).to(dtype)
    # Per-example scale so that some examples clip and some do not.
    x = x * torch.logspace(-1, 0.5, n).view(n, 1, 1).to(dtype)
    fz_d = to(frozen, DEV)
    prod_loss = model_loss(capture.peft_lora_linear, fz_d)
    ref_loss = model_loss(None, frozen)
    # Oracle on the CPU in float32 copies of the same values.
    if C is None:
        _, aux0 = dp_ref.clipped_grad(ref_loss, train, (x, y), clipping_norm=float("inf"))
        C = float(aux0["norms"].median())
    kw = dict(normalize_by=normalize_by, second_moment=second_moment, dtype=out_dtype)
    if autos:
        fn, st = auto_clipped_grad(prod_loss, R=C, batch_argnums=(1, 2), return_aux=return_aux,
                                   microbatch_size=microbatch, **kw)
    else:
        fn, st = clipped_grad(prod_loss, clipping_norm=C, batch_argnums=(1, 2), return_aux=return_aux,
                              microbatch_size=microbatch, **kw)
    out, st2 = fn(to(train, DEV), x.to(DEV), y.to(DEV), state=st)
    torch.cuda.synchronize()
    summed, aux = dp_ref.clipped_grad(ref_loss, train, (x, y), clipping_norm=C, autos=autos,
                                      normalize_by=normalize_by, second_moment=second_moment,
                                      dtype=out_dtype)
    run_both.last_fn = fn
    return out, st, st2, summed, aux, C


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("autos", [False, True])
def test_lora_capture_matches_oracle(dtype, tol, autos):
    out, st, st2, summed, aux, C = run_both(dtype, autos=autos)
    assert st2 is st
    grads, gaux = out
    assert isinstance(grads, ClippedPytree)
    assert grads.max_norm == C
    assert isinstance(gaux, AutoClippedGradAux if autos else ClippedGradAux)
    for k, ref in summed.items():
        got = grads.pytree[k]
        assert got.dtype == dtype and got.shape == ref.shape, k
        assert rel(got, ref) <= tol, (k, rel(got, ref))
    assert rel(gaux.grad_norms, aux["norms"]) <= tol
    assert rel(gaux.loss_values, aux["loss_values"]) <= tol
    assert rel(gaux.clipped_grad_norms, aux["clipped_norms"]) <= max(tol, 1e-5)
    assert gaux.batch_size == 6
    # The kernel's per-example clip masks (norm > C, AUTO-S counting the same
    # way) equal the oracle's for every example away from the threshold band,
    # and so does the clipping rate when no example lies in the band.
    band = 1e-3 if dtype == torch.bfloat16 else 1e-6
    ref_n = aux["norms"].double()
    far = ((ref_n - C).abs() / C) > band
    mask = run_both.last_fn.engine._plan.clipped_total.cpu().bool()
    assert torch.equal(mask[far], (ref_n > C)[far]), (mask, ref_n, C)
    assert 0 < int((ref_n[far] > C).sum()) < int(far.sum())  # both outcomes occur
    ref_rate = float((ref_n[far] > C).sum()) / len(ref_n)
    if bool(far.all()):
        assert gaux.clipping_rate == pytest.approx(ref_rate)


def test_capture_route_was_taken():
    frozen, train = make_model(torch.float32)
    fz_d = to(frozen, DEV)
    loss = model_loss(capture.peft_lora_linear, fz_d)
    fn, st = clipped_grad(loss, clipping_norm=1.0, batch_argnums=(1, 2))
    x = torch.randn(3, 8, 32, device=DEV)
    fn(to(train, DEV), x, x, state=st)
    disc = fn.engine._discovery[1]
    # All eight LoRA factors are captured at the seam; the norm weights are not.
    assert len(disc.eligible) == 8


def test_shared_factor_falls_back_to_materialised():
    frozen, train = make_model(torch.float32, layers=1)
    fz_d = to(frozen, DEV)

    def loss(params, x, y):
        a = params["l0.up.lora_A"]
        u = capture.peft_lora_linear(x, fz_d["l0.up.W"], a, params["l0.up.lora_B"], 2.0)
        # lora_A is also used outside the seam: its per-example gradient must
        # come from autograd, and the seam it feeds cannot be captured.
        u = u + (x @ a.t()).sum(-1, keepdim=True)
        v = capture.peft_lora_linear(torch.tanh(u), fz_d["l0.down.W"], params["l0.down.lora_A"],
                                     params["l0.down.lora_B"], 2.0)
        return ((v * params["l0.norm"] - y) ** 2).mean()

    def ref_loss(params, x, y):
        a = params["l0.up.lora_A"]
        u = _plain_lora(x, frozen["l0.up.W"], a.t(), params["l0.up.lora_B"].t(), 2.0)
        u = u + (x @ a.t()).sum(-1, keepdim=True)
        v = _plain_lora(torch.tanh(u), frozen["l0.down.W"], params["l0.down.lora_A"].t(),
                        params["l0.down.lora_B"].t(), 2.0)
        return ((v * params["l0.norm"] - y) ** 2).mean()

    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, 8, 32, generator=g)
    y = torch.randn(4, 8, 32, generator=g)
    fn, st = clipped_grad(loss, clipping_norm=0.5, batch_argnums=(1, 2))
    out, _ = fn(to(train, DEV), x.to(DEV), y.to(DEV), state=st)
    disc = fn.engine._discovery[1]
    assert len(disc.eligible) == 2  # only the down projection's factors
    ref, _ = dp_ref.clipped_grad(ref_loss, train, (x, y), clipping_norm=0.5)
    for k, r in ref.items():
        assert rel(out.pytree[k], r) <= 1e-5, k


def test_materialised_route_linear_regression():
    # The reference docstring example (_clipped_grad.py:112-129): theta = 3, data [0, 7, -2].
    def f(theta, d):
        return 0.5 * ((d - theta) ** 2).mean()

    fn, st = clipped_grad(f, clipping_norm=float("inf"), return_aux=True)
    (res, aux), _ = fn(torch.tensor(3.0, device=DEV), torch.tensor([0.0, 7.0, -2.0], device=DEV), state=st)
    # Per-example gradients 3, -4, 5 pass unclipped; their sum is 4 (mean 4/3).
    assert res.pytree.item() == pytest.approx(4.0, rel=1e-6)
    assert aux.loss_values.cpu().tolist() == pytest.approx([4.5, 8.0, 12.5])
    assert aux.grad_norms.cpu().tolist() == pytest.approx([3.0, 4.0, 5.0])
    fn3, st3 = clipped_grad(f, clipping_norm=float("inf"), normalize_by=3.0)
    res3, _ = fn3(torch.tensor(3.0, device=DEV), torch.tensor([0.0, 7.0, -2.0], device=DEV), state=st3)
    assert res3.pytree.item() == pytest.approx(4.0 / 3.0, rel=1e-6)
    assert res3.max_norm == math.inf


def test_materialised_route_matches_oracle_fixed_clip():
    g = torch.Generator().manual_seed(3)
    params = {"w": torch.randn(12, 5, generator=g), "b": torch.randn(5, generator=g)}
    x = torch.randn(9, 12, generator=g) * torch.logspace(-1, 1, 9).view(9, 1)
    y = torch.randn(9, 5, generator=g)

    def f(p, xi, yi):
        return ((xi @ p["w"] + p["b"] - yi) ** 2).sum()

    fn, st = clipped_grad(f, clipping_norm=3.0, batch_argnums=(1, 2), return_aux=True, normalize_by=4.0)
    (res, aux), _ = fn({k: v.to(DEV) for k, v in params.items()}, x.to(DEV), y.to(DEV), state=st)
    ref, raux = dp_ref.clipped_grad(f, params, (x, y), clipping_norm=3.0, normalize_by=4.0)
    for k in params:
        assert rel(res.pytree[k], ref[k]) <= 1e-5
    assert rel(aux.grad_norms, raux["norms"]) <= 1e-6
    assert res.max_norm == 3.0 / 4.0


def test_custom_scale_fn():
    """clipped_grad(_scale_fn=...) (_clipped_fun.py:660-700): the caller's
    per-example scaling replaces the built-in clip; the kernels sum the
    scaled gradients, the aux norms are the ones the function reports."""
    import types

    g = torch.Generator().manual_seed(5)
    params = {"w": torch.randn(12, 5, generator=g), "b": torch.randn(5, generator=g)}
    x = torch.randn(9, 12, generator=g) * torch.logspace(-1, 1, 9).view(9, 1)
    y = torch.randn(9, 5, generator=g)
    C = 30.0  # four of the nine examples exceed it

    def f(p, xi, yi):
        return ((xi @ p["w"] + p["b"] - yi) ** 2).sum()

    def halve_above(grad):  # a bounding scheme of the caller's: examples above C are halved
        nrm = torch.sqrt(sum((t.double() ** 2).sum() for t in grad.values()))
        s = torch.where(nrm > C, torch.full_like(nrm, 0.5), torch.ones_like(nrm))
        return {k: v * s.to(v.dtype) for k, v in grad.items()}, types.SimpleNamespace(norm=nrm, group_norms=None)

    # Expected on the CPU: per-example gradients, the same scaling, a float32 sum.
    pe = torch.func.vmap(torch.func.grad(f), in_dims=(None, 0, 0))(params, x, y)
    def tensors_only(grad):
        sc, rec = halve_above(grad)
        return sc, rec.norm

    scaled, norm = torch.func.vmap(tensors_only)(pe)
    want = {k: v.sum(0) / 4.0 for k, v in scaled.items()}
    want_cn = torch.sqrt(sum((v.double() ** 2).flatten(1).sum(1) for v in scaled.values()))

    pd = {k: v.to(DEV) for k, v in params.items()}
    fn, st = clipped_grad(f, clipping_norm=C, batch_argnums=(1, 2), return_aux=True, normalize_by=4.0,
                          _scale_fn=halve_above)
    (res, aux), _ = fn(pd, x.to(DEV), y.to(DEV), state=st)
    for k in params:
        assert rel(res.pytree[k], want[k]) <= 1e-5, k
    assert res.max_norm == C / 4.0
    assert rel(aux.grad_norms, norm) <= 1e-6  # the function's own norms (fp32 gradients on either side)
    assert rel(aux.clipped_grad_norms, want_cn) <= 1e-5
    above = int((norm > C).sum())
    assert 0 < above < 9
    assert aux.clipping_rate == pytest.approx(above / 9)
    fs, sst = clipped_grad(f, clipping_norm=C, batch_argnums=(1, 2), return_stats=True, _scale_fn=halve_above)
    (res2, stats), _ = fs(pd, x.to(DEV), y.to(DEV), state=sst)
    assert stats.num_clipped == float(above) and stats.batch_size == 9 and stats.all_finite
    for k in params:
        assert rel(res2.pytree[k], want[k] * 4.0) <= 1e-5, k


def test_custom_scale_fn_output_is_summed_as_it_is():
    """The reference sums a scale function's output as it is
    (_clipped_fun.py:673-700, 777-782): NaN entries it returns stay NaN in
    the sum, and values whose squares overflow float32 are still summed
    (their clipped norms are inf, not a reason to drop the example).  Here
    the function turns large entries into NaN and multiplies examples above
    C by 1e30."""
    import types

    g = torch.Generator().manual_seed(9)
    params = {"w": torch.randn(12, 5, generator=g), "b": torch.randn(5, generator=g)}
    x = torch.randn(9, 12, generator=g) * torch.logspace(-1, 1, 9).view(9, 1)
    y = torch.randn(9, 5, generator=g)
    C, T = 30.0, 40.0

    def f(p, xi, yi):
        return ((xi @ p["w"] + p["b"] - yi) ** 2).sum()

    def wild(grad):
        nrm = torch.sqrt(sum((t.double() ** 2).sum() for t in grad.values()))
        s = torch.where(nrm > C, torch.full_like(nrm, 1e30), torch.ones_like(nrm)).float()
        out = {k: torch.where(v.abs() > T, torch.full_like(v, float("nan")), v) * s for k, v in grad.items()}
        return out, types.SimpleNamespace(norm=nrm, group_norms=None)

    pe = torch.func.vmap(torch.func.grad(f), in_dims=(None, 0, 0))(params, x, y)
    scaled, norm = torch.func.vmap(lambda gr: (wild(gr)[0], wild(gr)[1].norm))(pe)
    want = {k: v.sum(0) / 4.0 for k, v in scaled.items()}
    # global_norm of the scaled gradient: float32 squares and sums.
    want_cn = torch.sqrt(sum((v.float() ** 2).flatten(1).sum(1) for v in scaled.values()))
    assert torch.isnan(want["w"]).any() and torch.isfinite(want["w"]).any()
    assert torch.isinf(want_cn).any() and torch.isfinite(want_cn).any()

    fn, st = clipped_grad(f, clipping_norm=C, batch_argnums=(1, 2), return_aux=True, normalize_by=4.0,
                          _scale_fn=wild)
    (res, aux), _ = fn({k: v.to(DEV) for k, v in params.items()}, x.to(DEV), y.to(DEV), state=st)
    for k in params:
        got, w = res.pytree[k].cpu(), want[k]
        assert torch.equal(torch.isnan(got), torch.isnan(w)), k
        fin = torch.isfinite(w)
        scale = w[fin].abs().max()
        assert ((got[fin] - w[fin]).abs() <= 1e-5 * w[fin].abs() + 1e-6 * scale).all(), k
    cn = aux.clipped_grad_norms.cpu().float()
    assert torch.equal(torch.isnan(cn), torch.isnan(want_cn)) and torch.equal(torch.isinf(cn), torch.isinf(want_cn))
    fin = torch.isfinite(want_cn)
    assert torch.allclose(cn[fin], want_cn[fin], rtol=1e-5)


def test_per_group_matches_oracle():
    frozen, train = make_model(torch.float32)
    pg = per_group(train, up=0.3, down=0.2, norm=0.5)
    fz_d = to(frozen, DEV)
    prod_loss = model_loss(capture.peft_lora_linear, fz_d)
    ref_loss = model_loss(None, frozen)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(5, 8, 32, generator=g)
    y = torch.randn(5, 8, 32, generator=g)
    fn, st = clipped_grad(prod_loss, clipping_norm=pg, batch_argnums=(1, 2), return_aux=True)
    (res, aux), _ = fn(to(train, DEV), x.to(DEV), y.to(DEV), state=st)
    ref, raux = dp_ref.clipped_grad(ref_loss, train, (x, y), clipping_norm=pg)
    assert isinstance(res.max_norm, PerGroup)
    for k in train:
        assert rel(res.pytree[k], ref[k]) <= 1e-5, k
    assert set(aux.group_norms) == set(raux["group_norms"])
    for name, v in raux["group_norms"].items():
        assert rel(aux.group_norms[name], v) <= 1e-5
    assert aux.clipping_rate is None


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_second_moment_microbatch_stats(dtype, tol):
    out, st, _, summed, aux, C = run_both(dtype, second_moment=True, normalize_by=2.0)
    res, _ = out
    assert isinstance(res, SecondMomentClippingOutput)
    assert res.squared_grads.max_norm == pytest.approx(C * C / 2.0)
    for k, ref in aux["squared"].items():
        assert rel(res.squared_grads.pytree[k], ref) <= tol, k
    for k, ref in summed.items():
        assert rel(res.grads.pytree[k], ref) <= tol, k
    if dtype != torch.float32:
        return
    # Microbatching gives the same sum.
    out_mb, _, _, summed_mb, _, _ = run_both(torch.float32, microbatch=4, return_aux=False, normalize_by=2.0)
    for k, ref in summed_mb.items():
        assert rel(out_mb.pytree[k], ref) <= 1e-5, k


def test_return_stats_and_output_dtype():
    frozen, train = make_model(torch.bfloat16)
    fz_d = to(frozen, DEV)
    loss = model_loss(capture.peft_lora_linear, fz_d)
    fn, st = clipped_grad(loss, clipping_norm=1e-3, batch_argnums=(1, 2), return_stats=True,
                          dtype=torch.float32)
    x = torch.randn(4, 8, 32, device=DEV, dtype=torch.bfloat16)
    (res, stats), _ = fn(to(train, DEV), x, x, state=st)
    assert isinstance(stats, ClippingStats)
    assert stats.batch_size == 4 and stats.num_clipped == 4.0 and stats.clipping_rate == 1.0
    assert stats.all_finite is True
    assert all(v.dtype == torch.float32 for v in res.pytree.values())


def test_empty_batch():
    fn, st = clipped_grad(lambda p, x: (p * x).sum(), clipping_norm=1.0, return_aux=True)
    p = torch.ones(3, device=DEV)
    (res, aux), _ = fn(p, torch.zeros(0, 3, device=DEV), state=st)
    assert torch.equal(res.pytree, torch.zeros(3, device=DEV))
    assert aux.batch_size == 0 and aux.clipping_rate == 0.0


@pytest.mark.parametrize("pe_bytes", [None, 0])
def test_full_weight_linear_seams_match_oracle(pe_bytes):
    """bf16 full-weight linears, per-group clipping.  pe_bytes None: the
    per-example weight gradients fit in HBM, so the outer-form norm kernel
    stores them and the clipped sum runs over storage; 0: nothing is stored,
    so the norms take the form with fewer flops at the measured kernel
    speeds (at these shapes the outer form: 1.6 * 48 * (64 + 96) is not
    below 2 * 64 * 96) and the clipped sum is the GEMM over prescaled
    activations.  The token-Gram kernels are covered in test_gpu_linear."""
    print(f"drop-in full-weight linears: linear_pe_bytes={pe_bytes}", flush=True)
    g = torch.Generator().manual_seed(21)
    d, h = 64, 96
    params = {
        "up.weight": (torch.randn(h, d, generator=g) / d**0.5).to(torch.bfloat16),
        "up.bias": torch.zeros(h, dtype=torch.bfloat16),
        "down.weight": (torch.randn(d, h, generator=g) / h**0.5).to(torch.bfloat16),
    }

    def make(lin):
        def loss(p, xi, yi):
            u = torch.nn.functional.gelu(lin(xi, p["up.weight"], p["up.bias"]))
            return ((lin(u, p["down.weight"], None).float() - yi.float()) ** 2).mean()

        return loss

    def plain(x, W, b):
        return torch.nn.functional.linear(x, W, b)

    n, T = 8, 48
    x = (torch.randn(n, T, d, generator=g) * torch.logspace(-1, 0.5, n).view(n, 1, 1)).to(torch.bfloat16)
    y = torch.randn(n, T, d, generator=g).to(torch.bfloat16)
    pg = per_group(params, up=0.05, down=0.08)
    fn, st = clipped_grad(make(capture.linear), clipping_norm=pg, batch_argnums=(1, 2), return_aux=True,
                          normalize_by=4.0)
    if pe_bytes is not None:
        fn.engine.plan_options["linear_pe_bytes"] = pe_bytes
    (res, aux), _ = fn({k: v.to(DEV) for k, v in params.items()}, x.to(DEV), y.to(DEV), state=st)
    disc = fn.engine._discovery[1]
    assert len(disc.eligible) == 2  # both weights captured; the bias is materialised
    ref, raux = dp_ref.clipped_grad(make(plain), params, (x, y), clipping_norm=pg, normalize_by=4.0)
    for k in params:
        assert rel(res.pytree[k], ref[k]) <= 2e-2, (k, rel(res.pytree[k], ref[k]))
    for name, v in raux["group_norms"].items():
        assert rel(aux.group_norms[name], v) <= 2e-2


@pytest.mark.parametrize("d,h,T,form", [(256, 384, 40, "gram"), (1024, 1024, 600, "gram256")])
def test_full_weight_gram_norms_through_the_drop_in(d, h, T, form):
    """Without room to store per-example gradients, short examples against
    wide weights make the engine take the token-Gram norms (the 128-row
    kernel below 512 rows, the 256-row-block kernel from 512 rows): the
    drop-in reaches them and still matches the oracle, group norms and
    per-example masks included."""
    from opaque_amd import _native as N

    print(f"drop-in Gram norms: d={d} h={h} T={T} ({form})", flush=True)
    g = torch.Generator().manual_seed(31)
    params = {"up": (torch.randn(h, d, generator=g) / d**0.5).to(torch.bfloat16),
              "down": (torch.randn(d, h, generator=g) / h**0.5).to(torch.bfloat16)}

    def make(lin):
        def loss(p, xi, yi):
            u = torch.nn.functional.gelu(lin(xi, p["up"], None))
            return ((lin(u, p["down"], None).float() - yi.float()) ** 2).mean()

        return loss

    def plain(x, W, b):
        return torch.nn.functional.linear(x, W, b)

    n = 4
    x = (torch.randn(n, T, d, generator=g) * torch.logspace(-1, 0.5, n).view(n, 1, 1)).to(torch.bfloat16)
    y = torch.randn(n, T, d, generator=g).to(torch.bfloat16)
    _, aux0 = dp_ref.clipped_grad(make(plain), params, (x, y), clipping_norm=float("inf"))
    C = float(aux0["norms"].median())
    fn, st = clipped_grad(make(capture.linear), clipping_norm=C, batch_argnums=(1, 2), return_aux=True,
                          normalize_by=float(n))
    fn.engine.plan_options["linear_pe_bytes"] = 0
    (res, aux), _ = fn({k: v.to(DEV) for k, v in params.items()}, x.to(DEV), y.to(DEV), state=st)
    plan = fn.engine._plan
    forms = {t[1] for t in plan.tables if t[0] == "lin_norm" and t[5] > 0 and t[1] != N.FORM_OUTER_GUARDED}
    assert forms == {N.FORM_GRAM if form == "gram" else N.FORM_GRAM256}, forms
    ref, raux = dp_ref.clipped_grad(make(plain), params, (x, y), clipping_norm=C, normalize_by=float(n))
    for k in params:
        assert rel(res.pytree[k], ref[k]) <= 2e-2, (k, rel(res.pytree[k], ref[k]))
    assert rel(aux.grad_norms, raux["norms"]) <= 2e-2
    ref_n = raux["norms"].double()
    far = ((ref_n - C).abs() / C) > 1e-3
    assert torch.equal(plan.clipped_total.cpu().bool()[far], (ref_n > C)[far])


@pytest.mark.parametrize("pe_bytes", [None, 0])
def test_full_weight_second_moment_matches_oracle(pe_bytes):
    """clipped_grad(second_moment=True) over bf16 full-weight seams: the
    reference squares every clipped per-example gradient and sums the squares
    (_clipped_fun.py:675-683,777-782).  pe_bytes None: stored gradients and
    the scale-sum; 0: nothing stored, the moments kernel forms each example's
    gradient tile on the fly.  Both moments rel 2e-2 vs the oracle, group
    norms rel 2e-2, per-example clip masks equal away from the threshold."""
    print(f"drop-in full-weight second moment: linear_pe_bytes={pe_bytes}", flush=True)
    g = torch.Generator().manual_seed(23)
    d, h, n, T = 64, 96, 8, 40
    params = {"up": (torch.randn(h, d, generator=g) / d**0.5).to(torch.bfloat16),
              "down": (torch.randn(d, h, generator=g) / h**0.5).to(torch.bfloat16)}

    def make(lin):
        def loss(p, xi, yi):
            u = torch.nn.functional.gelu(lin(xi, p["up"], None))
            return ((lin(u, p["down"], None).float() - yi.float()) ** 2).mean()

        return loss

    def plain(x, W, b):
        return torch.nn.functional.linear(x, W, b)

    x = (torch.randn(n, T, d, generator=g) * torch.logspace(-1, 0.5, n).view(n, 1, 1)).to(torch.bfloat16)
    y = torch.randn(n, T, d, generator=g).to(torch.bfloat16)
    pg = per_group(params, up=0.05, down=0.08)
    fn, st = clipped_grad(make(capture.linear), clipping_norm=pg, batch_argnums=(1, 2), return_aux=True,
                          normalize_by=4.0, second_moment=True)
    if pe_bytes is not None:
        fn.engine.plan_options["linear_pe_bytes"] = pe_bytes
    (out, aux), _ = fn({k: v.to(DEV) for k, v in params.items()}, x.to(DEV), y.to(DEV), state=st)
    assert len(fn.engine._discovery[1].eligible) == 2
    tables = {t[0] for t in fn.engine._plan.tables if t[5] > 0}
    assert ("lin_moments" in tables) == (pe_bytes == 0), tables
    ref, raux = dp_ref.clipped_grad(make(plain), params, (x, y), clipping_norm=pg, normalize_by=4.0,
                                    second_moment=True)
    for k in params:
        assert rel(out.grads.pytree[k], ref[k]) <= 2e-2, (k, rel(out.grads.pytree[k], ref[k]))
        assert rel(out.squared_grads.pytree[k], raux["squared"][k]) <= 2e-2, k
    for name, v in raux["group_norms"].items():
        assert rel(aux.group_norms[name], v) <= 2e-2
        thr = {"up": 0.05, "down": 0.08}[name]
        far = ((v.double() - thr).abs() / thr) > 1e-3
        got = aux.group_norms[name].cpu() > thr
        assert torch.equal(got[far], (v > thr)[far]), name


@pytest.mark.parametrize("pe_bytes", [None, 0])
def test_full_weight_non_finite_activation(pe_bytes):
    """A NaN in one example's activations: the reference zeroes the non-finite
    entries of that example's weight gradient (nan_to_num,
    clipping/_pytree.py:520-527) and reports all_finite=False
    (_clipped_fun.py:98-112,695); a clean batch reports True."""
    print(f"drop-in non-finite activation: linear_pe_bytes={pe_bytes}", flush=True)
    g = torch.Generator().manual_seed(5)
    d, h, n, T = 64, 96, 6, 40
    params = {"w": (torch.randn(h, d, generator=g) / d**0.5).to(torch.bfloat16)}

    def make(lin):
        def loss(p, xi, yi):
            return (lin(xi, p["w"], None).float() * yi.float()).sum() / T

        return loss

    def plain(x, W, b):
        return torch.nn.functional.linear(x, W, b)

    x = torch.randn(n, T, d, generator=g).to(torch.bfloat16)
    y = torch.randn(n, T, h, generator=g).to(torch.bfloat16)
    for bad in (False, True):
        xb = x.clone()
        if bad:
            xb[2, 11, 5] = float("nan")
        fn, st = clipped_grad(make(capture.linear), clipping_norm=0.5, batch_argnums=(1, 2), return_stats=True)
        if pe_bytes is not None:
            fn.engine.plan_options["linear_pe_bytes"] = pe_bytes
        (res, stats), _ = fn({k: v.to(DEV) for k, v in params.items()}, xb.to(DEV), y.to(DEV), state=st)
        assert len(fn.engine._discovery[1].eligible) == 1
        assert stats.all_finite is (not bad)
        assert torch.isfinite(res.pytree["w"].float()).all()
        ref, _ = dp_ref.clipped_grad(make(plain), params, (xb, y), clipping_norm=0.5)
        assert rel(res.pytree["w"], ref["w"]) <= 2e-2, rel(res.pytree["w"], ref["w"])
