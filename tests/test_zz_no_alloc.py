"""The allocation-free entry point against the two entry points it replaces.

odp_clip_materialized_noalloc (partials in the library's static device
array) must give bit-identical scales, norms and masks to odp_sqnorm into a
caller buffer followed by odp_clip_factors, on two calls in a row (the
second smaller, so stale partials of the first would show), and refuse a
problem larger than its array before launching anything.  A table whose
slot runs past the partials has that write dropped by the kernel's own
bounds check, and the call reports NaN norms and zero scales; the next
valid call is unaffected.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from opaque_amd import _native as N

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _case(n_ex, sizes, dtypes, seed):
    """Materialised per-example leaves and the odp_sqnorm table over them (one
    segment per example), slots laid out leaf by leaf, leaves in two groups."""
    lib = N.load()
    g = torch.Generator().manual_seed(seed)
    leaves, rows, blocks, keep = [], [], [], []
    slot = 0
    group_end = []
    for k, (n, dt) in enumerate(zip(sizes, dtypes)):
        x = (torch.randn(n_ex, n, generator=g) * (1 + k)).to(dt).to(DEV)
        if k == 1:
            x[1, 3] = float("nan")  # counted as 0, as the reference's nan_to_num does
        leaves.append(x)
        nb = int(lib.odp_sqnorm_blocks(n))
        rows.append([x.data_ptr(), n, n_ex, 0, slot, {torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16}[dt],
                     0, 0])
        blocks.append(n_ex * nb)
        slot += nb
        group_end.append(slot)
    n_slots = slot
    probs = torch.tensor(np.asarray(rows, dtype=np.int64), device=DEV)
    ws = torch.tensor(np.concatenate([[0], np.cumsum(blocks)]).astype(np.int32), device=DEV)
    seg_ex = torch.arange(n_ex, dtype=torch.int32, device=DEV)
    gstart = torch.tensor([0, group_end[0], n_slots], dtype=torch.int64, device=DEV)
    return dict(probs=probs, ws=ws, n_prob=len(rows), total=int(sum(blocks)), seg_ex=seg_ex, n_slots=n_slots,
                n_ex=n_ex, gstart=gstart, keep=leaves)


def _outputs(n_ex):
    return dict(scale=torch.full((2, 2, n_ex), -1.0, dtype=torch.float64, device=DEV),
                norm=torch.full((n_ex,), -1.0, device=DEV), gnorm=torch.full((2, n_ex), -1.0, device=DEV),
                clip=torch.full((2, n_ex), 7, dtype=torch.uint8, device=DEV),
                clip_t=torch.full((n_ex,), 7, dtype=torch.uint8, device=DEV))


def _clip_args(c, o, thr, guard, cls):
    return (c["gstart"].data_ptr(), 2, thr.data_ptr(), 2.5, N.CLIP_FIXED, 0.0, 2, guard.data_ptr(),
            cls.data_ptr(), o["scale"].data_ptr(), o["norm"].data_ptr(), o["gnorm"].data_ptr(),
            o["clip"].data_ptr(), o["clip_t"].data_ptr())


def test_noalloc_matches_sqnorm_then_clip_factors():
    thr = torch.tensor([1.5, 2.0], dtype=torch.float64, device=DEV)
    guard = torch.tensor([1 - 2**-8, 1e-40, 1 - 2**-23, 1e-44], dtype=torch.float64, device=DEV)
    cls = torch.tensor([N.DTYPE_BF16, N.DTYPE_F32], dtype=torch.int32, device=DEV)
    for call, (n_ex, sizes) in enumerate([(7, [300, 9000, 17, 64]), (3, [40, 11])]):
        print(f"no-alloc call {call}: n_ex={n_ex} sizes={sizes}", flush=True)
        dts = [torch.float32, torch.bfloat16, torch.float32, torch.bfloat16][: len(sizes)]
        c = _case(n_ex, sizes, dts, seed=call)
        a, b = _outputs(n_ex), _outputs(n_ex)
        part = torch.zeros(n_ex, c["n_slots"], dtype=torch.float64, device=DEV)
        N.call("odp_sqnorm", _stream(), c["probs"].data_ptr(), c["ws"].data_ptr(), c["n_prob"], c["total"],
               c["seg_ex"].data_ptr(), part.data_ptr(), c["n_slots"])
        N.call("odp_clip_factors", _stream(), part.data_ptr(), c["n_slots"], n_ex, *_clip_args(c, a, thr, guard, cls))
        N.call("odp_clip_materialized_noalloc", _stream(), c["probs"].data_ptr(), c["ws"].data_ptr(), c["n_prob"],
               c["total"], c["seg_ex"].data_ptr(), c["n_slots"], n_ex, *_clip_args(c, b, thr, guard, cls))
        torch.cuda.synchronize()
        for k in a:
            assert torch.equal(a[k], b[k]), (call, k, a[k], b[k])
        assert (a["norm"] > 0).all() and (a["scale"] >= 0).all()


def test_noalloc_refuses_problems_beyond_its_array():
    lib = N.load()
    cap = int(lib.odp_noalloc_max_partials())
    assert cap == 1 << 20
    thr = torch.tensor([1.0], dtype=torch.float64, device=DEV)
    dummy = torch.zeros(8, dtype=torch.float64, device=DEV)
    gs = torch.tensor([0, cap], dtype=torch.int64, device=DEV)
    rc = lib.odp_clip_materialized_noalloc(_stream(), None, None, 0, 0, None, cap, 2, gs.data_ptr(), 1,
                                           thr.data_ptr(), 1.0, N.CLIP_FIXED, 0.0, 1, dummy.data_ptr(),
                                           gs.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), None, None, None)
    assert rc == N.ERR_UNSUPPORTED
    assert "static scratch" in N.last_error()


def test_noalloc_drops_writes_outside_its_partials():
    thr = torch.tensor([1.5, 2.0], dtype=torch.float64, device=DEV)
    guard = torch.tensor([1 - 2**-8, 1e-40, 1 - 2**-23, 1e-44], dtype=torch.float64, device=DEV)
    cls = torch.tensor([N.DTYPE_BF16, N.DTYPE_F32], dtype=torch.int32, device=DEV)
    c = _case(3, [40, 11], [torch.float32, torch.bfloat16], seed=5)
    bad = c["probs"].clone()
    bad[1, 4] = c["n_slots"]  # the second leaf's slot: one past the last partial of a row
    print("no-alloc: slot past the partials", flush=True)
    o = _outputs(3)
    N.call("odp_clip_materialized_noalloc", _stream(), bad.data_ptr(), c["ws"].data_ptr(), c["n_prob"],
           c["total"], c["seg_ex"].data_ptr(), c["n_slots"], 3, *_clip_args(c, o, thr, guard, cls))
    torch.cuda.synchronize()
    assert torch.isnan(o["norm"]).all() and torch.isnan(o["gnorm"]).all()
    assert (o["scale"] == 0).all() and (o["clip"] == 0).all() and (o["clip_t"] == 0).all()
    # The status is cleared by the next call, which matches the caller-buffer path.
    a, b = _outputs(3), _outputs(3)
    part = torch.zeros(3, c["n_slots"], dtype=torch.float64, device=DEV)
    N.call("odp_sqnorm", _stream(), c["probs"].data_ptr(), c["ws"].data_ptr(), c["n_prob"], c["total"],
           c["seg_ex"].data_ptr(), part.data_ptr(), c["n_slots"])
    N.call("odp_clip_factors", _stream(), part.data_ptr(), c["n_slots"], 3, *_clip_args(c, a, thr, guard, cls))
    N.call("odp_clip_materialized_noalloc", _stream(), c["probs"].data_ptr(), c["ws"].data_ptr(), c["n_prob"],
           c["total"], c["seg_ex"].data_ptr(), c["n_slots"], 3, *_clip_args(c, b, thr, guard, cls))
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k
