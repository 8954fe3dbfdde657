"""float16 / bfloat16 / float32 / float64 leaves through the drop-in ``clipped_grad``.

Ports the reference's dtype sweep (opaque-engine/tests/clipping/
test_clipping_numerics.py:24-85,113-124): for every dtype, tree shape and
gradient magnitude, the clipped gradient *as stored* has norm <= C with no
tolerance (a batch of one example, so the output is that example's clipped
gradient), and a batch matches the CPU oracle.  The per-example gradient is
the example's own data (loss = sum(p * x)), so every value is exact.

Tolerances against the oracle: float64 rel 1e-12, float32 1e-6, 16-bit
dtypes 2e-2 (the clip scale is bit-exact given the same squared norm; the
norms' fp64 summation order may differ in the last place, which can move a
16-bit scale by one unit).
"""

from __future__ import annotations

import pytest
import torch

from opaque_amd.clipping import auto_clipped_grad, clipped_grad
from oracle import dp_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
LOW = [torch.bfloat16, torch.float16]
ALL = [*LOW, torch.float32, torch.float64]
NORM_SCALES = [1e-3, 1.0, 1e2, 1e4, 1e6]
TREES = {
    "scalar": lambda g, d: {"a": torch.randn((), generator=g).to(d)},
    "vector": lambda g, d: {"a": torch.randn(17, generator=g).to(d)},
    "matrix": lambda g, d: {"a": torch.randn(8, 12, generator=g).to(d)},
    "nested": lambda g, d: {"enc": {"w": torch.randn(5, 3, generator=g).to(d)},
                            "dec": {"w": torch.randn(7, generator=g).to(d), "b": torch.zeros(2, dtype=d)}},
    "ragged": lambda g, d: {f"p{i}": torch.randn(i + 1, generator=g).to(d) for i in range(6)},
}


def _leaves(tree):
    return [x for _, x in dp_ref.flatten(tree)]


def _loss(p, x):
    tot = None
    for a, b in zip(_leaves(p), _leaves(x)):
        t = (a * b).sum().double()
        tot = t if tot is None else tot + t
    return tot


def _exact_norm(tree) -> float:
    return float(sum((t.double() ** 2).sum() for t in _leaves(tree)) ** 0.5)


def _to(tree, dev):
    return dp_ref.rebuild(tree, {p: x.to(dev) for p, x in dp_ref.flatten(tree)})


def _zeros_like(tree):
    return dp_ref.rebuild(tree, {p: torch.zeros_like(x) for p, x in dp_ref.flatten(tree)})


@pytest.mark.parametrize("dtype", ALL)
@pytest.mark.parametrize("shape", list(TREES))
def test_bound_holds_as_stored(dtype, shape):
    print(f"dtype sweep: bound as stored {dtype} {shape}", flush=True)
    g = torch.Generator().manual_seed(0)
    for mag in NORM_SCALES:
        for C in (0.01, 1.0, 7.5):
            x = TREES[shape](g, dtype)
            x = dp_ref.rebuild(x, {p: (t * mag).to(dtype) for p, t in dp_ref.flatten(x)})
            fn, st = clipped_grad(_loss, clipping_norm=C)
            batch = dp_ref.rebuild(x, {p: t.unsqueeze(0) for p, t in dp_ref.flatten(x)})
            res, _ = fn(_to(_zeros_like(x), DEV), _to(batch, DEV), state=st)
            for a in _leaves(res.pytree):
                assert a.dtype == dtype
            assert _exact_norm(res.pytree) <= C, (dtype, shape, mag, C)


@pytest.mark.parametrize("dtype", ALL)
def test_auto_scale_bound_holds_as_stored(dtype):
    """AUTO-S has no min(1, .), so the bound rests on the guard alone (:88-97)."""
    g = torch.Generator().manual_seed(1)
    for mag in NORM_SCALES:
        for R in (0.01, 1.0, 7.5):
            x = {"w": (torch.randn(64, generator=g) * mag).to(dtype)}
            fn, st = auto_clipped_grad(_loss, R=R, gamma=0.01)
            res, _ = fn(_to(_zeros_like(x), DEV), {"w": x["w"].unsqueeze(0).to(DEV)}, state=st)
            assert _exact_norm(res.pytree) <= R, (dtype, mag, R)


@pytest.mark.parametrize("low", LOW)
def test_mixed_dtype_tree_bound_holds(low):
    """A low-precision and a float64 leaf in one tree (:113-124); the float64
    leaf makes float64 the accumulation dtype of the whole call."""
    g = torch.Generator().manual_seed(3)
    for mag in NORM_SCALES:
        x = {"low": (torch.randn(20, generator=g) * mag).to(low),
             "high": (torch.randn(20, generator=g) * mag).double()}
        fn, st = clipped_grad(_loss, clipping_norm=1.0)
        res, _ = fn(_to(_zeros_like(x), DEV), {k: v.unsqueeze(0).to(DEV) for k, v in x.items()}, state=st)
        assert res.pytree["low"].dtype == low and res.pytree["high"].dtype == torch.float64
        assert _exact_norm(res.pytree) <= 1.0


@pytest.mark.parametrize("dtype", ALL)
@pytest.mark.parametrize("autos", [False, True])
def test_batch_matches_oracle(dtype, autos):
    """Six examples, normalize_by 3: norms, clipped sum and dtypes against the oracle."""
    print(f"dtype sweep: batch vs oracle {dtype} autos={autos}", flush=True)
    g = torch.Generator().manual_seed(7)
    params = {"a": torch.zeros(9, 4, dtype=dtype), "b": torch.zeros(33, dtype=dtype)}
    xs = {"a": (torch.randn(6, 9, 4, generator=g) * torch.logspace(-1, 1, 6).view(6, 1, 1)).to(dtype),
          "b": (torch.randn(6, 33, generator=g) * 0.5).to(dtype)}
    C = 2.0
    if autos:
        fn, st = auto_clipped_grad(_loss, R=C, gamma=0.01, normalize_by=3.0, return_aux=True)
    else:
        fn, st = clipped_grad(_loss, clipping_norm=C, normalize_by=3.0, return_aux=True)
    (res, aux), _ = fn(_to(params, DEV), _to(xs, DEV), state=st)
    want, waux = dp_ref.clipped_grad(_loss, params, (xs,), clipping_norm=C, normalize_by=3.0, autos=autos)
    tol = {torch.float64: 1e-12, torch.float32: 1e-6}.get(dtype, 2e-2)
    for k in params:
        got = res.pytree[k]
        assert got.dtype == dtype
        w = want[k].double()
        assert (got.double().cpu() - w).norm() <= tol * w.norm(), (k, dtype)
    assert torch.allclose(aux.grad_norms.double().cpu(), waux["norms"].double(), rtol=max(tol, 1e-6))


def test_float64_compute_dtype_with_float32_leaves():
    """compute_dtype=float64: squares and the batch sum in float64
    (_pytree.py:81-103, _clipped_fun.py:115-134)."""
    g = torch.Generator().manual_seed(11)
    params = {"w": torch.zeros(300, dtype=torch.float32)}
    xs = {"w": torch.randn(5, 300, generator=g) * torch.logspace(-2, 2, 5).view(5, 1)}
    fn, st = clipped_grad(_loss, clipping_norm=1.5, compute_dtype=torch.float64, normalize_by=2.0)
    res, _ = fn(_to(params, DEV), _to(xs, DEV), state=st)
    want, _ = dp_ref.clipped_grad(_loss, params, (xs,), clipping_norm=1.5, normalize_by=2.0,
                                  compute_dtype=torch.float64)
    assert res.pytree["w"].dtype == torch.float32
    w = want["w"].double()
    assert (res.pytree["w"].double().cpu() - w).norm() <= 1e-7 * w.norm()
