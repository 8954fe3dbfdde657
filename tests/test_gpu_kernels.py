"""GPU parity of the native kernels against the CPU oracle (needs an MI355X)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from opaque_amd import _native as N
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LoraSite, MaterializedLeaf, Segments
from opaque_amd.guard import guard_constants, leaf_guards
from oracle import lora_ref, philox_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stream():
    return torch.cuda.current_stream().cuda_stream


def test_philox_device_matches_known_answers():
    out = torch.empty((1, 4), dtype=torch.int32, device=DEV)
    for ctr, key, want in philox_ref.KAT:
        c0 = ctr[0] | (ctr[1] << 32)
        seed = key[0] | (key[1] << 32)
        N.call("odp_philox_words", _stream(), c0, ctr[2], ctr[3], seed, 1, out.data_ptr())
        got = tuple(int(v) & 0xFFFFFFFF for v in out.cpu().view(-1).tolist())
        assert got == want


def test_philox_device_matches_oracle_stream():
    n = 4096
    seed = 0x0123456789ABCDEF
    out = torch.empty((n, 4), dtype=torch.int32, device=DEV)
    N.call("odp_philox_words", _stream(), 2**32 - 7, 5, 0, seed, n, out.data_ptr())
    got = out.cpu().numpy().view(np.uint32)
    ctr = np.arange(2**32 - 7, 2**32 - 7 + n, dtype=np.uint64)
    want = philox_ref.philox4x32_10(ctr & np.uint64(0xFFFFFFFF), ctr >> np.uint64(32), 5, 0,
                                    seed & 0xFFFFFFFF, seed >> 32)
    np.testing.assert_array_equal(got, np.stack(want, axis=-1))


def _lora_case(dtype, n_ex, T, d_in, d_out, r, lengths=None, seed=0, scaling=2.0):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(n_ex * T, d_in, generator=g).to(dtype)
    G = torch.randn(n_ex * T, d_out, generator=g).to(dtype)
    A = (torch.randn(d_in, r, generator=g) / math.sqrt(d_in)).to(dtype)
    B = (torch.randn(r, d_out, generator=g) * 0.02).to(dtype)
    seg = Segments.padded(n_ex, T, lengths)
    return X, G, A, B, seg, scaling


def _run_single_site(X, G, A, B, seg, scaling, C=1.0, mode=N.CLIP_FIXED, normalize_by=1.0):
    dt = X.dtype
    shapes = [tuple(A.shape), tuple(B.shape)]
    acc, rnd = leaf_guards(shapes, [dt, dt])
    rel, ab = guard_constants(dt, rnd)
    leaves = [LeafOut(tuple(A.shape), dt), LeafOut(tuple(B.shape), dt)]
    site = LoraSite(X.to(DEV), G.to(DEV), A.to(DEV), B.to(DEV), scaling, a_leaf=0, b_leaf=1)
    clip = ClipSpec(mode=mode, thresholds=[C], effective=C, normalize_by=normalize_by, guards=[(rel, ab, dt)])
    plan = GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=[site], device=DEV)
    res = plan.run()
    torch.cuda.synchronize()
    return plan, res


@pytest.mark.parametrize(
    "dtype,n_ex,T,d_in,d_out,r,lengths",
    [
        (torch.float32, 4, 64, 96, 80, 8, None),
        (torch.float32, 3, 40, 128, 64, 16, [40, 17, 0]),
        (torch.bfloat16, 4, 64, 256, 128, 16, None),
        (torch.bfloat16, 5, 96, 136, 264, 8, [96, 33, 1, 70, 64]),
        (torch.bfloat16, 2, 128, 512, 384, 48, [128, 100]),
        (torch.bfloat16, 3, 64, 200, 72, 64, [64, 20, 5]),
        (torch.float32, 2, 48, 104, 96, 32, None),
        (torch.bfloat16, 2, 32, 72, 40, 4, None),
    ],
)
def test_lora_norms_and_factor_grads(dtype, n_ex, T, d_in, d_out, r, lengths):
    X, G, A, B, seg, s = _lora_case(dtype, n_ex, T, d_in, d_out, r, lengths)
    plan, res = _run_single_site(X, G, A, B, seg, s, C=1e30)
    dA, dB = lora_ref.lora_per_example(X, G, A, B, s, seg.starts, seg.lengths)
    want = (dA.pow(2).sum((1, 2)) + dB.pow(2).sum((1, 2))).sqrt()
    got = res.norms.double().cpu()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert torch.allclose(got, want, rtol=tol, atol=1e-30), (got, want)
    # C huge: nothing clipped, so the sum equals sum_i dA_i (in leaf layout).
    sa = dA.sum(0)
    sb = dB.sum(0)
    ga, gb = res.leaves[0].double().cpu(), res.leaves[1].double().cpu()
    assert (ga - sa).norm() <= tol * sa.norm() + 1e-12
    assert (gb - sb).norm() <= tol * sb.norm() + 1e-12


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", [N.CLIP_FIXED, N.CLIP_AUTOS])
def test_clipped_sum_matches_oracle(dtype, mode):
    X, G, A, B, seg, s = _lora_case(dtype, 6, 48, 128, 96, 8, [48, 20, 33, 48, 5, 41], seed=3)
    dA, dB = lora_ref.lora_per_example(X, G, A, B, s, seg.starts, seg.lengths)
    norms = (dA.pow(2).sum((1, 2)) + dB.pow(2).sum((1, 2))).sqrt()
    C = float(norms.median())  # about half the examples clip
    plan, res = _run_single_site(X, G, A, B, seg, s, C=C, mode=mode, normalize_by=6.0)
    if mode == N.CLIP_FIXED:
        fac = torch.clamp(C / norms, max=1.0)
    else:
        fac = C / (norms + 0.01)
    wa = (fac[:, None, None] * dA).sum(0) / 6.0
    wb = (fac[:, None, None] * dB).sum(0) / 6.0
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    # fp32: the reference guard shrinks the scale by ~1e-7 relative; bf16 by ~0.8%.
    ga, gb = res.leaves[0].double().cpu(), res.leaves[1].double().cpu()
    assert (ga - wa).norm() <= tol * wa.norm()
    assert (gb - wb).norm() <= tol * wb.norm()
    # saturation mask is exact away from the threshold
    got_mask = res.clipped_total.cpu().bool()
    want_mask = norms.float() > C
    band = 1e-6 if dtype == torch.float32 else 1e-3
    far = ((norms - C).abs() / C) > band
    assert torch.equal(got_mask[far], want_mask[far])


def test_clip_factor_arithmetic_is_bit_exact():
    """Given identical squared norms, the device scale equals the oracle's torch fp64 chain."""
    from oracle import dp_ref

    sq = torch.tensor([0.0, 1e-30, 0.25, 1.0, 1.0000001, 4.0, 1e6, float("inf"), 2.5e-3, 9.0], dtype=torch.float64)
    n = sq.numel()
    part = sq.reshape(n, 1).to(DEV)
    for C, mode in [(1.0, N.CLIP_FIXED), (0.7, N.CLIP_FIXED), (float("inf"), N.CLIP_FIXED), (1.0, N.CLIP_AUTOS)]:
        for store in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
            rnd = dp_ref.roundoff(torch.float64 if store == torch.float64 else torch.float32, 7, 3000)
            rel, ab = guard_constants(store, rnd)
            gs = torch.tensor([0, 1], dtype=torch.int64, device=DEV)
            thr = torch.tensor([C], dtype=torch.float64, device=DEV)
            guard = torch.tensor([rel, ab], dtype=torch.float64, device=DEV)
            code = {torch.float32: N.DTYPE_F32, torch.bfloat16: N.DTYPE_BF16, torch.float16: N.DTYPE_F16,
                    torch.float64: N.DTYPE_F64}[store]
            cls = torch.tensor([code], dtype=torch.int32, device=DEV)
            scale = torch.empty((1, 1, n), dtype=torch.float64, device=DEV)
            norms = torch.empty(n, dtype=torch.float32, device=DEV)
            gn = torch.empty((1, n), dtype=torch.float32, device=DEV)
            cl = torch.empty((1, n), dtype=torch.uint8, device=DEV)
            ct = torch.empty(n, dtype=torch.uint8, device=DEV)
            N.call("odp_clip_factors", _stream(), part.data_ptr(), 1, n, gs.data_ptr(), 1, thr.data_ptr(), C,
                   mode, 0.01, 1, guard.data_ptr(), cls.data_ptr(), scale.data_ptr(), norms.data_ptr(),
                   gn.data_ptr(), cl.data_ptr(), ct.data_ptr())
            torch.cuda.synchronize()
            nrm = torch.sqrt(sq)
            c_t = torch.clamp(torch.tensor(C, dtype=torch.float64), min=0.0)
            ratio = c_t / (nrm + 0.01) if mode == N.CLIP_AUTOS else c_t / nrm
            want = dp_ref.finalize(ratio, store, rnd, mode == N.CLIP_FIXED).to(store).double()
            assert torch.equal(scale.view(-1).cpu(), want), (C, mode, store, scale.view(-1).cpu(), want)
            assert torch.equal(norms.cpu(), nrm.float())
            assert torch.equal(ct.cpu().bool(), nrm.float() > C)


def test_clip_factors_take_partials_at_any_8_byte_offset():
    """The partials may start 8 bytes past a 16-byte boundary (a sub-view of
    a caller's buffer): the pair loads follow the address, and the result
    equals that of an aligned copy up to the fp64 summation order."""
    g = torch.Generator().manual_seed(2)
    n_ex, n_slots = 5, 1001
    sq = torch.rand(n_ex, n_slots, generator=g, dtype=torch.float64)
    base = torch.zeros(n_ex * n_slots + 2, dtype=torch.float64, device=DEV)
    out = {}
    for off in (0, 1):
        part = base[off : off + n_ex * n_slots]
        part.copy_(sq.reshape(-1).to(DEV))
        assert (part.data_ptr() % 16 == 8) == (off == 1)
        gs = torch.tensor([0, 400, n_slots], dtype=torch.int64, device=DEV)
        thr = torch.tensor([10.0, 12.0], dtype=torch.float64, device=DEV)
        guard = torch.tensor([1.0 - 2**-23, 0.0], dtype=torch.float64, device=DEV)
        cls = torch.tensor([N.DTYPE_F32], dtype=torch.int32, device=DEV)
        scale = torch.empty((1, 2, n_ex), dtype=torch.float64, device=DEV)
        norms = torch.empty(n_ex, dtype=torch.float32, device=DEV)
        gn = torch.empty((2, n_ex), dtype=torch.float32, device=DEV)
        N.call("odp_clip_factors", _stream(), part.data_ptr(), n_slots, n_ex, gs.data_ptr(), 2, thr.data_ptr(),
               15.6, N.CLIP_FIXED, 0.0, 1, guard.data_ptr(), cls.data_ptr(), scale.data_ptr(), norms.data_ptr(),
               gn.data_ptr(), None, None)
        torch.cuda.synchronize()
        out[off] = (gn.double().cpu(), scale.cpu())
    want = torch.stack([sq[:, :400].sum(1), sq[:, 400:].sum(1)]).sqrt()
    for off in (0, 1):
        assert torch.allclose(out[off][0], want, rtol=1e-6)
    assert torch.allclose(out[0][1], out[1][1], rtol=1e-6)


@pytest.mark.parametrize("dt,shape", [(torch.float32, (3, 7)), (torch.bfloat16, (3, 7)),
                                      (torch.bfloat16, (6, 40)), (torch.float32, (5, 48))])
def test_materialized_leaf_path(dt, shape):
    """Odd sizes take the scale-sum's element-wise path, multiples of 8 its vector path."""
    print(f"materialized leaf: {dt} {shape}", flush=True)
    g = torch.Generator().manual_seed(5)
    pe = torch.randn(5, *shape, generator=g).to(dt)  # 5 examples of the leaf
    seg = Segments.padded(5, 1)
    acc, rnd = leaf_guards([shape], [dt])
    rel, ab = guard_constants(dt, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[2.0], effective=2.0, guards=[(rel, ab, dt)])
    plan = GhostPlan(segments=seg, leaves=[LeafOut(shape, dt)], clip=clip,
                     materialized=[MaterializedLeaf(pe.to(DEV), 0)], device=DEV)
    res = plan.run()
    torch.cuda.synchronize()
    from oracle import dp_ref

    outs, norms = [], []
    for i in range(5):
        c, nrm, _ = dp_ref.clip_pytree({"w": pe[i]}, 2.0)
        outs.append(c["w"].float())
        norms.append(nrm)
    want = torch.stack(outs).sum(0).to(dt)
    tol = 1e-6 if dt == torch.float32 else 2e-2
    got = res.leaves[0].cpu()
    assert got.dtype == dt and got.shape == shape
    assert torch.allclose(got.float(), want.float(), rtol=tol, atol=tol)
    assert torch.allclose(res.norms.cpu(), torch.stack(norms).float(), rtol=1e-6 if dt == torch.float32 else 1e-5)


def test_noise_kernel_matches_oracle_and_is_deterministic():
    from opaque_amd.noise import add_noise_tree

    g = torch.Generator().manual_seed(0)
    tree = {"a": torch.randn(1000, 3, generator=g), "b": torch.randn(777, generator=g)}
    dev_tree = {k: v.to(DEV) for k, v in tree.items()}
    seed = 0xDEADBEEFCAFEF00D
    out1 = add_noise_tree(dev_tree, 0.8, seed)
    out2 = add_noise_tree(dev_tree, 0.8, seed)
    out3 = add_noise_tree(dev_tree, 0.8, seed + 1)
    torch.cuda.synchronize()
    for k in tree:
        assert torch.equal(out1[k], out2[k])
        assert not torch.equal(out1[k], out3[k])
    # sorted-key flat offsets: "a" first (3000 elements), then "b"
    wa = philox_ref.gaussian_noise(tree["a"].numpy(), 0.8, seed, 0)
    wb = philox_ref.gaussian_noise(tree["b"].numpy(), 0.8, seed, 3000)
    np.testing.assert_allclose(out1["a"].cpu().numpy().reshape(-1), wa, rtol=2e-6, atol=2e-6)
    np.testing.assert_allclose(out1["b"].cpu().numpy().reshape(-1), wb, rtol=2e-6, atol=2e-6)


def test_noise_statistics():
    from scipy import stats

    from opaque_amd.noise import add_noise_tree

    z = torch.zeros(1_000_000, device=DEV)
    out = add_noise_tree({"z": z}, 1.0, 12345)["z"].cpu().double().numpy()
    assert abs(out.mean()) < 5e-3
    assert abs(out.std() - 1.0) < 5e-3
    assert stats.kstest(out[:100_000], "norm").pvalue > 0.01
    bf = add_noise_tree({"z": torch.zeros(100_000, device=DEV, dtype=torch.bfloat16)}, 2.5, 7)["z"]
    assert bf.dtype == torch.bfloat16
    assert abs(bf.float().std().item() - 2.5) < 0.05
