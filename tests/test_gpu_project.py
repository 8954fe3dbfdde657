"""odp_project called directly through the C ABI: Q^T[k][row] = sum_j P[row][j] W[k][j].

The bf16 projection streams P and W into LDS and accumulates in fp32 on the
matrix cores, then rounds to bf16.  Its workgroups walk the covered rows
(each segment widened to whole 8-row groups): every covered row must equal
the float64 product of the same bf16 operands rounded to bf16, within one
bf16 unit in the last place (the fp32 sum may sit on the other side of a
rounding boundary), and every other row must be left as it was.  The grid
is sized from the covered rows (odp_project_covered_rows) or, as an upper
bound, from all rows.  fp32 P walks all rows: rows in segments match at
fp32 tolerance and all others are 0, including the rows of blocks that
hold no segment row.  Shapes cover every rank block count (1..4), ranks
that are not multiples of 16, contraction lengths that are not multiples of
the 64-column step, row counts that are not multiples of the 256-row block,
ragged and unaligned segments (two of them sharing an 8-row group), and a
table of two problems.
"""

from __future__ import annotations

import pytest
import torch

from opaque_amd import _native as N

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (n_rows, d, [r per problem], segments as (start, length))
CASES = [
    (1000, 4096, [16], [(0, 300), (512, 488)]),
    (777, 200, [40], [(0, 777)]),
    (300, 136, [64], [(10, 50), (100, 200)]),
    (2048, 1024, [8, 13], [(0, 1024), (1300, 700)]),
    (1200, 520, [32, 20], [(700, 100)]),  # rows 0..511 and 1024.. hold no segment row
    (900, 328, [40, 48], [(3, 250), (253, 13), (266, 0), (270, 601), (880, 20)]),  # unaligned, shared group
    (37, 24, [16], [(5, 1), (9, 20)]),  # a contraction shorter than one step, a one-row segment
    (300, 64, [16], []),  # no segment at all
]


def _covered(n_rows, segs):
    cov = torch.zeros(n_rows, dtype=torch.bool)
    for s, n in segs:
        if n > 0:
            cov[s & ~7:min((s + n + 7) & ~7, n_rows)] = True
    return cov


def _ref(P: torch.Tensor, W: torch.Tensor, rows: torch.Tensor, dtype) -> torch.Tensor:
    full = (P.double() @ W.double().t()).t()  # [r][n_rows]
    return torch.where(rows[None, :], full, torch.zeros_like(full)).to(dtype)


def _run(n_rows, d, ranks, segs, dtype, seed, tight=False):
    lib = N.load()
    g = torch.Generator(device=DEV).manual_seed(seed)
    ldp = d + 24  # a row pitch wider than the contraction
    P = torch.randn(n_rows, ldp, device=DEV, generator=g).to(dtype)
    ldq = (n_rows + 32 + 7) // 8 * 8
    nkb = (max(ranks) + 15) // 16
    Ws, Qs = [], []
    for r in ranks:
        assert (r + 15) // 16 == nkb
        Ws.append((torch.randn(r, d, device=DEV, generator=g) / d ** 0.5).to(dtype))
        # Planes start out as NaN, so that an unwritten entry shows.
        Qs.append(torch.full((16 * nkb, ldq), float("nan"), device=DEV, dtype=dtype))
    sst = torch.tensor([s for s, _ in segs] or [0], device=DEV, dtype=torch.int32)
    sln = torch.tensor([n for _, n in segs] or [0], device=DEV, dtype=torch.int32)
    code = N.DTYPE_BF16 if dtype == torch.bfloat16 else N.DTYPE_F32
    walk = n_rows
    if tight:
        hs = torch.tensor([s for s, _ in segs] or [0], dtype=torch.int32)
        hl = torch.tensor([n for _, n in segs] or [0], dtype=torch.int32)
        walk = int(lib.odp_project_covered_rows(hs.data_ptr(), hl.data_ptr(), len(segs)))
        assert walk == sum(((s + n + 7) & ~7) - (s & ~7) for s, n in segs if n > 0)
    per = int(lib.odp_project_blocks(code, walk, max(ranks)))
    rows = []
    for W, Q, r in zip(Ws, Qs, ranks):
        row = [0] * N.PJ_FIELDS
        row[N.PJ_P], row[N.PJ_LDP], row[N.PJ_D] = P.data_ptr(), ldp, d
        row[N.PJ_W], row[N.PJ_R], row[N.PJ_Q], row[N.PJ_LDQ] = W.data_ptr(), r, Q.data_ptr(), ldq
        row[N.PJ_NROWS], row[N.PJ_SEG_FIRST], row[N.PJ_NSEG] = n_rows, 0, len(segs)
        rows.append(row)
    probs = torch.tensor(rows, dtype=torch.int64).view(-1).to(DEV)
    ws = torch.tensor([per * i for i in range(len(ranks) + 1)], dtype=torch.int32, device=DEV)
    print(f"odp_project: rows {n_rows} d {d} ranks {ranks} nkb {nkb} {dtype}", flush=True)
    rc = lib.odp_project(torch.cuda.current_stream().cuda_stream, code, probs.data_ptr(), ws.data_ptr(),
                         len(ranks), per * len(ranks), sst.data_ptr(), sln.data_ptr(), nkb)
    N.check(rc, "odp_project")
    torch.cuda.synchronize()
    inside = torch.zeros(n_rows, dtype=torch.bool, device=DEV)
    for s, n in segs:
        inside[s:s + n] = True
    if dtype == torch.bfloat16:
        inside = _covered(n_rows, segs).to(DEV)
    return [(Q[:r, :n_rows], _ref(P[:, :d], W, inside, dtype), inside) for W, Q, r in zip(Ws, Qs, ranks)]


@pytest.mark.parametrize("tight", [True, False])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_bf16_projection(case, tight):
    n_rows, d, ranks, segs = CASES[case]
    for got, want, inside in _run(n_rows, d, ranks, segs, torch.bfloat16, seed=case, tight=tight):
        assert torch.isnan(got[:, ~inside]).all(), "rows outside the covered groups were written"
        assert not torch.isnan(got[:, inside]).any(), "covered rows left unwritten"
        if not inside.any():
            continue
        g, w = got[:, inside].float(), want[:, inside].float()
        # One bf16 ulp of the reference: 2^(e - 8) for frexp's exponent e.
        ulp = torch.ldexp(torch.ones_like(w), torch.frexp(w)[1] - 8)
        bad = (g - w).abs() > ulp
        assert not bad.any(), (bad.sum().item(), (g - w).abs().max().item())
        assert (g == w).float().mean() > 0.95


@pytest.mark.parametrize("case", [0, 2, 3, 5, 6, 7])
def test_f32_projection(case):
    n_rows, d, ranks, segs = CASES[case]
    for got, want, inside in _run(n_rows, d, ranks, segs, torch.float32, seed=10 + case):
        assert not torch.isnan(got).any(), "unwritten plane entries"
        assert (got[:, ~inside] == 0).all()
        torch.testing.assert_close(got[:, inside], want[:, inside], rtol=1e-5, atol=1e-5)
