"""The streamed factor pass (odp_seg_factor_stream) against the tiled one
(odp_seg_factor with the same number of rank blocks).

Both form a problem's per-example rows pe[k][m] = scaling * sum_t Q[k][t]
P[t][m] from the same 32-token MFMA blocks in the same order, then square
and store the same bf16 values into the same partial slots, so every output
of a plan must be bit-identical with the streamed pass on and off:
per-example rows, norms, scales, clip masks and clipped sums.  Covered: dB
rows from G and V, dA rows from X and U (a one-site activation, the per-site
rows of sites with different scalings, and activations shared by two or
three sites of rank 16, one of them with a frozen A: a rank block without a
leaf), the mirrored order of a down projection, sites bringing the seam's V
and U, widths that split a segment's tiles into several groups with a
partial last tile, empty, single-row, longest and unaligned segments, and
the cases that keep the tiled pass (leaves off the 16-row blocks, a segment
past the length limit).
"""

from __future__ import annotations

import math

import pytest
import torch

from opaque_amd import _native as N
from opaque_amd.engine import ClipSpec, GhostPlan, LeafOut, LoraSite, Segments
from opaque_amd.guard import guard_constants, leaf_guards

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _sites(n_rows, d_in, outs, ranks, frozen=(), scalings=None, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    X = torch.randn(n_rows, d_in, device=DEV, generator=g).to(torch.bfloat16)
    sites, leaves = [], []
    for i, (d_out, r) in enumerate(zip(outs, ranks)):
        G = (torch.randn(n_rows, d_out, device=DEV, generator=g) * 0.3).to(torch.bfloat16)
        A = (torch.randn(d_in, r, device=DEV, generator=g) / math.sqrt(d_in)).to(torch.bfloat16)
        B = (torch.randn(r, d_out, device=DEV, generator=g) * 0.05).to(torch.bfloat16)
        ia = ib = None
        if (i, "A") not in frozen:
            ia = len(leaves)
            leaves.append(LeafOut(tuple(A.shape), torch.bfloat16))
        if (i, "B") not in frozen:
            ib = len(leaves)
            leaves.append(LeafOut(tuple(B.shape), torch.bfloat16))
        sc = 2.0 if scalings is None else scalings[i]
        sites.append(LoraSite(X, G, A, B, sc, a_leaf=ia, b_leaf=ib))
    return sites, leaves


def _plan(seg, sites, leaves, stream, C, fuse=True):
    shapes = [lf.shape for lf in leaves]
    _, rnd = leaf_guards(shapes, [torch.bfloat16] * len(shapes))
    rel, ab = guard_constants(torch.bfloat16, rnd)
    clip = ClipSpec(mode=N.CLIP_FIXED, thresholds=[C], effective=C, normalize_by=2.0,
                    guards=[(rel, ab, torch.bfloat16)])
    return GhostPlan(segments=seg, leaves=leaves, clip=clip, lora_sites=sites, device=DEV,
                     stream_factors=stream, fuse_g_side=fuse)


def _outputs(plan):
    res = plan.run()
    torch.cuda.synchronize()
    out = [t.clone() for t in plan.pe_views()] + [t.clone() for t in res.leaves]
    return out + [res.norms.clone(), res.scales.clone(), res.clipped.clone()]


def _compare(seg, sites, leaves, expect_stream=True, fuse=True):
    """expect_stream: whether the plan must hold streamed rows (None: either)."""
    base = _plan(seg, sites, leaves, False, 1e30, fuse)
    norms = base.run().norms.double().cpu()
    torch.cuda.synchronize()
    C = float(norms[norms > 0].median()) if (norms > 0).any() else 1.0  # some examples clipped, some not
    off = _plan(seg, sites, leaves, False, C, fuse)
    on = _plan(seg, sites, leaves, True, C, fuse)
    live_on = {t[0] for t in on.tables if t[5] > 0}
    live_off = {t[0] for t in off.tables if t[5] > 0}
    assert "factor_stream" not in live_off
    if expect_stream is not None:
        assert ("factor_stream" in live_on) == expect_stream, live_on
    want, got = _outputs(off), _outputs(on)
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), k
    return on


CASES = [
    # n_ex, T, lengths, d_in, d_outs, ranks, frozen
    (5, 96, [96, 33, 1, 70, 64], 136, [264], [8], ()),             # partial last tile, length 1
    (3, 1081, [1081, 0, 517], 64, [512], [16], ()),                # longest segment, empty segment
    (4, 40, [40, 39, 17, 25], 96, [1000, 200], [12, 4], ()),       # two sites on one X: dA stays tiled
    (3, 64, [64, 50, 9], 128, [256, 136], [8, 8], ((0, "B"), (1, "A"))),  # frozen factors
    (4, 80, [80, 33, 1, 64], 520, [136], [16], ()),                # mirrored: d_in > d_out
    (3, 200, [200, 0, 57], 264, [4360], [16], ()),                 # 18 tiles in several groups, partial last
    (2, 129, [129, 88], 4360, [8200], [16], ()),                   # dA over 18 tiles, dB over 33 (uneven groups)
    (3, 128, [128, 77, 0], 256, [256, 64, 64], [16, 16, 16], ()),  # q/k/v: dA in three rank blocks
    (3, 128, [128, 5, 90], 256, [256, 64, 64], [16, 16, 8], ((1, "A"),)),  # a rank block without a leaf
    (3, 96, [96, 50, 3], 128, [512, 512], [16, 8], ()),            # gate/up: two rank blocks, rank 8 last
]


@pytest.mark.parametrize("fuse", [True, False])
@pytest.mark.parametrize("n_ex,T,lengths,d_in,d_outs,ranks,frozen", CASES)
def test_streamed_factor_rows_equal_tiled(n_ex, T, lengths, d_in, d_outs, ranks, frozen, fuse):
    """With the fused G side off every dB row streams; with it on, the dA
    rows of one-leaf activations and the dB rows of mirrored sites do."""
    print(f"factor stream: n_ex={n_ex} T={T} d_in={d_in} d_outs={d_outs} ranks={ranks} fuse={fuse}", flush=True)
    seg = Segments.padded(n_ex, T, lengths)
    sites, leaves = _sites(n_ex * T, d_in, d_outs, ranks, frozen)
    _compare(seg, sites, leaves, expect_stream=None if fuse else True, fuse=fuse)


def test_sites_with_different_scalings_stream_their_own_da_rows():
    print("factor stream: per-site dA rows (different scalings)", flush=True)
    seg = Segments.padded(3, 72, [72, 40, 5])
    sites, leaves = _sites(3 * 72, 200, [96, 264], [16, 8], scalings=[2.0, 0.5])
    _compare(seg, sites, leaves)


def test_unaligned_segments():
    print("factor stream: packed segments at unaligned starts", flush=True)
    lengths = [13, 37, 77, 0, 100]
    starts = [0, 13, 50, 127, 127]
    seg = Segments(starts, lengths, list(range(5)), 5, 240)
    sites, leaves = _sites(240, 72, [328], [16], seed=5)
    _compare(seg, sites, leaves)


def test_segment_past_the_limit_keeps_the_tiled_pass():
    limit = int(N.load().odp_factor_project_max_len())
    T = limit + 21
    print(f"factor stream: segment of {T} rows (limit {limit})", flush=True)
    seg = Segments.padded(2, T, [T, 40])
    sites, leaves = _sites(2 * T, 96, [200], [16], seed=7)
    _compare(seg, sites, leaves, expect_stream=False)


@pytest.mark.parametrize("shared", [False, True])
def test_seam_products(shared):
    """Sites bringing V and U: every dB row and the dA rows of one-site
    activations take the streamed pass."""
    print(f"factor stream: seam products, shared activation={shared}", flush=True)
    seg = Segments.padded(4, 96, [96, 0, 41, 77])
    outs, ranks = ([256, 64, 64], [16, 16, 8]) if shared else ([4360], [16])
    sites, leaves = _sites(4 * 96, 512 if not shared else 256, outs, ranks, seed=3)
    proj = _plan(seg, sites, leaves, False, 1.0)
    proj.run()
    torch.cuda.synchronize()
    with_vu = []
    for i, s in enumerate(sites):
        v, u = proj.rank_planes(i)
        with_vu.append(LoraSite(s.x, s.g, s.A, s.B, s.scaling, a_leaf=s.a_leaf, b_leaf=s.b_leaf,
                                v=v.contiguous(), u=u.contiguous()))
    on = _compare(seg, with_vu, leaves)
    live = {t[0] for t in on.tables if t[5] > 0}
    assert "planes" in live and not live & {"project", "factor_project", "factor"}, live
    keys = {t[1] for t in on.tables if t[0] == "factor_stream" and t[5] > 0}
    assert keys == ({1, 3} if shared else {1}), keys


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


@pytest.mark.parametrize("entry", ["stream", "fused"])
def test_segment_past_the_limit_gets_nan_partials(entry):
    """Called directly (the engine never does this) with a segment longer
    than the single-pass kernels hold (odp_factor_project_max_len() rows
    whatever the alignment; 17 steps of 64 rows from an 8-aligned start),
    every partial slot of that example becomes NaN and the other segment's
    slots are computed as usual."""
    lib = N.load()
    limit = int(lib.odp_factor_project_max_len())
    lens = [limit + 8, 40]  # 1089 rows from row 0: 18 steps
    starts = [0, limit + 1]
    n_rows = sum(lens)
    print(f"factor {entry}: segment of {lens[0]} rows (limit {limit})", flush=True)
    M, r = 512, 16
    ldq = (n_rows + 32 + 7) // 8 * 8
    g = torch.Generator(device=DEV).manual_seed(9)
    P = torch.randn(n_rows, M, device=DEV, generator=g).to(torch.bfloat16)
    Q = torch.randn(32, ldq, device=DEV, generator=g).to(torch.bfloat16)  # rows 16.. are read, not used
    W = torch.randn(r, M, device=DEV, generator=g).to(torch.bfloat16)
    U = torch.zeros(32, ldq, device=DEV, dtype=torch.bfloat16)
    pe = torch.zeros(2, r, M, device=DEV, dtype=torch.bfloat16)
    tiles = int(lib.odp_seg_factor_tiles(N.DTYPE_BF16, M, r))
    n_slots = N.FT_WAVE_SLOTS * tiles
    part = torch.zeros(2, n_slots, device=DEV, dtype=torch.float64)
    sst = torch.tensor(starts, device=DEV, dtype=torch.int32)
    sln = torch.tensor(lens, device=DEV, dtype=torch.int32)
    sex = torch.tensor([0, 1], device=DEV, dtype=torch.int32)
    rows = []
    for j in range(2):
        row = [0] * N.FT_FIELDS
        row[N.FT_P], row[N.FT_LDP], row[N.FT_M] = _ptr(P), M, M
        row[N.FT_Q], row[N.FT_LDQ], row[N.FT_R] = _ptr(Q), ldq, r
        row[N.FT_SEG_FIRST], row[N.FT_NSEG] = j, 1
        row[N.FT_SCALING] = int(torch.tensor([2.0], dtype=torch.float64).view(torch.int64).item())
        row[N.FT_NLEAF] = 1
        row[N.FT_LEAF0] = _ptr(pe) + j * r * M * 2
        row[N.FT_LEAF0 + 1] = 0 | (r << 16) | (1 << 32)
        row[N.FT_LEAF0 + 2] = 0
        if entry == "fused":
            row[N.FP_W], row[N.FP_U] = _ptr(W), _ptr(U)
        else:
            row[N.FT_GROUPS] = int(lib.odp_seg_factor_stream_groups(M))
        rows.append(row)
    probs = torch.tensor(rows, dtype=torch.int64).view(-1).to(DEV)
    per = 1 if entry == "fused" else int(lib.odp_seg_factor_stream_groups(M))
    ws = torch.tensor([0, per, 2 * per], dtype=torch.int32, device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    if entry == "fused":
        rc = lib.odp_seg_factor_project(s, _ptr(probs), _ptr(ws), 2, 2 * per, _ptr(sst), _ptr(sln), _ptr(sex),
                                        _ptr(part), n_slots)
    else:
        rc = lib.odp_seg_factor_stream(s, _ptr(probs), _ptr(ws), 2, 2 * per, _ptr(sst), _ptr(sln), _ptr(sex),
                                       _ptr(part), n_slots, 1)
    N.check(rc, entry)
    torch.cuda.synchronize()
    assert torch.isnan(part[0]).all(), part[0]
    assert torch.isfinite(part[1]).all() and (part[1] > 0).any(), part[1]
    # The short segment's squared norm: the sum of squares of its stored rows.
    want = pe[1].float().square().double().sum()
    assert torch.allclose(part[1].sum(), want, rtol=1e-9), (part[1].sum(), want)
