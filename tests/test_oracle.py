"""The CPU oracle against the reference's known answers, invariants and brute force.

Runs without a GPU.  The golden vectors are the reference tests' own
expected values (tests/golden/reference_vectors.json, each case citing its
source); the invariants are the ones the reference's numerics tests assert.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import dp_ref, lora_ref, philox_ref

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "reference_vectors.json")) as _f:
    CASES = {c["name"]: c for c in json.load(_f)["cases"]}


class _Groups:
    """Minimal PerGroup stand-in for the oracle: path tuple -> group, group -> value."""

    def __init__(self, groups: dict, values: dict) -> None:
        self.groups = groups
        self.values = values


def _tree(obj):
    if isinstance(obj, dict):
        return {k: _tree(v) for k, v in obj.items()}
    return torch.tensor(obj, dtype=torch.float32)


def _groups_for(case, tree):
    if "groups" in case:
        return _Groups({(k,): g for k, g in case["groups"].items()}, dict(case["values"]))
    if "patterns" in case:
        groups = {}
        for path, _ in dp_ref.flatten(tree):
            display = ".".join(str(p) for p in path)
            hits = [p for p in case["patterns"] if p in display]
            assert len(hits) == 1
            groups[path] = hits[0]
        return _Groups(groups, dict(case["patterns"]))
    return None


def _assert_tree_close(got, expected, rtol):
    for path, t in dp_ref.flatten(got):
        exp = expected
        for p in path:
            exp = exp[p]
        exp_t = torch.tensor(exp, dtype=torch.float64)
        if rtol == 0.0:
            assert torch.equal(t.double(), exp_t), (path, t, exp_t)
        else:
            torch.testing.assert_close(t.double(), exp_t, rtol=rtol, atol=1e-7)


@pytest.mark.parametrize("name", [n for n, c in CASES.items() if c["kind"] in ("clip", "auto")])
def test_oracle_clip_golden(name):
    case = CASES[name]
    tree = _tree(case["tree"])
    pg = _groups_for(case, tree)
    if case["kind"] == "clip":
        out, norm, gnorms = dp_ref.clip_pytree(tree, pg)
    else:
        R = pg if pg is not None else case["R"]
        out, norm, gnorms = dp_ref.auto_scale_pytree(tree, R, case["gamma"])
    if "expected" in case:
        _assert_tree_close(out, case["expected"], case["rtol"])
    if "expected_norm" in case:
        assert norm.item() == pytest.approx(case["expected_norm"], rel=1e-7, abs=0.0)
    if "expected_group_norms" in case:
        for g, v in case["expected_group_norms"].items():
            assert gnorms[g].item() == pytest.approx(v, rel=1e-6)
    if "expected_output_norm" in case:
        assert dp_ref.global_norm(out).item() == pytest.approx(case["expected_output_norm"], rel=case["rtol"])


def test_oracle_global_norm_golden():
    case = CASES["global_norm_13"]
    assert dp_ref.global_norm(_tree(case["tree"])).item() == case["expected_norm"]


def test_oracle_clipped_grad_docstring():
    case = CASES["clipped_grad_docstring"]

    def f(theta, d):
        return 0.5 * ((d - theta) ** 2).mean()

    summed, aux = dp_ref.clipped_grad(f, torch.tensor(case["theta"]), (torch.tensor(case["data"]),),
                                      clipping_norm=float("inf"))
    assert aux["loss_values"].tolist() == case["expected_loss_values"]
    assert aux["norms"].tolist() == case["expected_grad_norms"]
    assert summed.item() == case["expected_sum"]
    mean, _ = dp_ref.clipped_grad(f, torch.tensor(case["theta"]), (torch.tensor(case["data"]),),
                                  clipping_norm=float("inf"), normalize_by=3.0)
    assert mean.item() == pytest.approx(4.0 / 3.0)


def test_oracle_per_group_sigma_golden():
    case = CASES["noise_per_group_sigma"]
    got = dp_ref.per_group_sigma(case["values"], case["noise_multiplier"])
    for k, v in case["expected"].items():
        assert got[k] == pytest.approx(v, rel=1e-12)


# ---------------------------------------------------------------------------
# Invariants of the clip arithmetic (test_clipping_numerics.py:61-190 in the reference)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("autos", [False, True])
def test_oracle_bound_holds_as_stored(dtype, autos):
    g = torch.Generator().manual_seed(7)
    for trial in range(20):
        tree = {
            "a": (torch.randn(37, 5, generator=g) * 10 ** (trial % 5 - 2)).to(dtype),
            "b": (torch.randn(5000, generator=g) * 10 ** (trial % 3 - 1)).to(dtype),
            "c": torch.randn(3, generator=g).to(dtype),
        }
        C = 0.37
        if autos:
            out, _, _ = dp_ref.auto_scale_pytree(tree, C, 0.01)
        else:
            out, _, _ = dp_ref.clip_pytree(tree, C)
        stored = math.sqrt(sum(float((t.double() ** 2).sum()) for _, t in dp_ref.flatten(out)))
        assert stored <= C, (dtype, trial, stored)


def test_oracle_passthrough_and_zero():
    tree = {"a": torch.tensor([1e-3, -2e-3]), "b": torch.tensor([[5e-4]])}
    out, norm, _ = dp_ref.clip_pytree(tree, 1.0)
    for (_, x), (_, y) in zip(dp_ref.flatten(out), dp_ref.flatten(tree)):
        assert torch.equal(x, y)
    zero, _, _ = dp_ref.clip_pytree(tree, 0.0)
    assert all(torch.equal(t, torch.zeros_like(t)) for _, t in dp_ref.flatten(zero))
    inf, _, _ = dp_ref.clip_pytree({"a": torch.tensor([3.0, 4.0])}, float("inf"))
    assert torch.equal(inf["a"], torch.tensor([3.0, 4.0]))


def test_oracle_fp32_guard_is_negligible():
    tree = {"a": torch.tensor([30.0, 40.0])}
    out, _, _ = dp_ref.clip_pytree(tree, 1.0)
    torch.testing.assert_close(out["a"], torch.tensor([0.6, 0.8]), rtol=1e-6, atol=0)


# The reference documents what its guard costs a clipped output (the
# AUTO-S and clip_pytree docstrings, _pytree.py:384-385,492-493): "~0.8% of
# the output magnitude at bfloat16, ~0.1% at float16 and ~1.2e-7 at float32",
# i.e. one unit roundoff of the storage dtype (2^-7, 2^-10, 2^-23) plus twice
# the norm roundoff.  Pinned from both sides, so that a guard made smaller
# (the bound could break) or larger (outputs shrink for nothing) fails.
GUARD_SHRINK = {torch.bfloat16: 2.0**-7, torch.float16: 2.0**-10, torch.float32: 2.0**-23}


@pytest.mark.parametrize("dt", list(GUARD_SHRINK))
@pytest.mark.parametrize("shapes", [[(3,)], [(8192, 16), (16, 4096)], [(4096, 16)] * 448])
def test_oracle_guard_magnitude_matches_reference_docs(dt, shapes):
    leaves = [torch.zeros(s, dtype=dt) for s in shapes]
    acc = dp_ref.acc_dtype(leaves, None)
    rnd = dp_ref.roundoff(acc, len(leaves), dp_ref.reduction_terms(leaves))
    # The norm roundoff is float32 squares plus float64 sums: a few parts in
    # 1e8 at most for these trees, far below the storage term.
    assert 0 < rnd < 1e-7
    ratio = torch.tensor([2.0, 0.37, 5.0e3], dtype=torch.float64)
    shrink = 1.0 - dp_ref.finalize(ratio, dt, rnd, clamp_one=False) / ratio
    eps = GUARD_SHRINK[dt]
    tiny = torch.finfo(dt).smallest_normal * torch.finfo(dt).eps / 0.37
    assert ((shrink - eps).abs() <= 2 * rnd + tiny + 1e-15).all(), (shrink, eps, rnd)
    # The storage term as the docstrings round it: 0.8 %, 0.1 %, 1.2e-7 (at
    # float32 the norm roundoff, 2 rnd ~ 6e-8, is of the same order and not
    # included in the documented figure).
    doc = {torch.bfloat16: 0.008, torch.float16: 0.001, torch.float32: 1.2e-7}[dt]
    assert abs((float(shrink[0]) - 2 * rnd) / doc - 1.0) < 0.03


def test_oracle_clipped_count_counts_strictly_above():
    """num_clipped = #(norm > C) (_clipped_fun.py:512-523): equality is not
    clipped; the count is taken in the norms' own dtype."""
    norms = torch.tensor([0.5, 1.0, 1.00000001, 3.0, float("inf")], dtype=torch.float64)
    assert dp_ref.clipped_count(norms, 1.0) == 3
    assert dp_ref.clipped_count(norms.float(), 1.0) == 2  # 1.00000001 rounds to 1.0 in float32
    assert dp_ref.clipped_count(torch.zeros(0), 1.0) == 0
    assert dp_ref.clipped_count(norms, float("inf")) == 0


def test_oracle_nan_sanitised():
    out, norm, _ = dp_ref.auto_scale_pytree({"a": torch.tensor([float("nan"), float("inf"), 1.0])}, 1.0, 0.01)
    assert torch.isfinite(out["a"]).all()
    assert norm.item() == 1.0


# ---------------------------------------------------------------------------
# Brute force: explicit per-example loop vs the oracle's vmap path
# ---------------------------------------------------------------------------


def test_oracle_clipped_grad_matches_explicit_loop():
    g = torch.Generator().manual_seed(1)
    params = {"w": torch.randn(6, 3, generator=g), "b": torch.randn(3, generator=g)}
    X = torch.randn(7, 6, generator=g) * torch.logspace(-1, 1, 7).view(7, 1)
    Y = torch.randn(7, 3, generator=g)

    def f(p, x, y):
        return ((x @ p["w"] + p["b"] - y) ** 2).sum()

    C = 2.0
    summed, aux = dp_ref.clipped_grad(f, params, (X, Y), clipping_norm=C, second_moment=True)
    first = {k: torch.zeros_like(v, dtype=torch.float64) for k, v in params.items()}
    second = {k: torch.zeros_like(v, dtype=torch.float64) for k, v in params.items()}
    for i in range(7):
        p = {k: v.clone().double().requires_grad_() for k, v in params.items()}
        loss = f(p, X[i].double(), Y[i].double())
        grads = torch.autograd.grad(loss, [p["b"], p["w"]])
        gi = {"b": grads[0], "w": grads[1]}
        norm = math.sqrt(sum(float((t**2).sum()) for t in gi.values()))
        assert aux["norms"][i].item() == pytest.approx(norm, rel=1e-6)
        s = min(1.0, C / norm)
        for k in gi:
            first[k] += s * gi[k]
            second[k] += (s * gi[k]) ** 2
    for k in params:
        torch.testing.assert_close(summed[k].double(), first[k], rtol=2e-6, atol=1e-6)
        torch.testing.assert_close(aux["squared"][k].double(), second[k], rtol=2e-6, atol=1e-6)


def test_lora_oracle_matches_autograd_per_example():
    g = torch.Generator().manual_seed(2)
    d_in, d_out, r, s = 12, 10, 4, 2.0
    X = torch.randn(9, d_in, generator=g, dtype=torch.float64)
    G = torch.randn(9, d_out, generator=g, dtype=torch.float64)
    A = torch.randn(d_in, r, generator=g, dtype=torch.float64)
    B = torch.randn(r, d_out, generator=g, dtype=torch.float64)
    starts, lengths = [0, 4], [4, 5]
    dA, dB = lora_ref.lora_per_example(X, G, A, B, s, starts, lengths)
    for i, (st, ln) in enumerate(zip(starts, lengths)):
        a = A.clone().requires_grad_()
        b = B.clone().requires_grad_()
        y = s * (X[st : st + ln] @ a) @ b
        ga, gb = torch.autograd.grad((y * G[st : st + ln]).sum(), [a, b])
        torch.testing.assert_close(dA[i], ga)
        torch.testing.assert_close(dB[i], gb)


def test_gram_identity():
    g = torch.Generator().manual_seed(3)
    X = torch.randn(11, 7, generator=g)
    G = torch.randn(11, 5, generator=g)
    starts, lengths = [0, 3, 3], [3, 0, 8]
    pe = lora_ref.linear_per_example(X, G, starts, lengths)
    gram = lora_ref.linear_sqnorm_gram(X, G, starts, lengths)
    torch.testing.assert_close((pe**2).sum(dim=(1, 2)), gram, rtol=1e-12, atol=1e-12)
    assert gram[1].item() == 0.0


# ---------------------------------------------------------------------------
# Philox and the noise transform
# ---------------------------------------------------------------------------


def test_philox_known_answers():
    for ctr, key, expect in philox_ref.KAT:
        out = philox_ref.philox4x32_10(*[np.uint64(c) for c in ctr], np.uint64(key[0]), np.uint64(key[1]))
        assert tuple(int(o) for o in out) == expect


def test_philox_noise_transform_statistics():
    z = philox_ref.gaussian_noise(np.zeros(200_000), 1.0, seed=1234, flat_offset=0)
    assert abs(z.mean()) < 0.01
    assert abs(z.std() - 1.0) < 0.01
    from scipy import stats

    assert stats.kstest(z, "norm").pvalue > 0.01


def test_fold_in_variadic_equals_sequential():
    k = dp_ref.key_seed(42)
    assert dp_ref.fold_in_seed(dp_ref.fold_in_seed(k, 7), 3) == dp_ref.fold_in_seed(k, 7, 3)
    assert dp_ref.fold_in_seed(k, "noise") != dp_ref.fold_in_seed(k, "sampling")


# ---------------------------------------------------------------------------
# fold_in: known answers from the byte format of ENG/random/_engine.py:27-35
# (each part as a 16-byte little-endian signed int, or UTF-8 text, followed
# by b"|"; BLAKE2b with an 8-byte digest read little-endian).  The expected
# values hash literal byte strings, so a width, sign, byte-order or
# separator slip in the restatement fails.
# ---------------------------------------------------------------------------

FOLD_IN_KAT = [
    # (seed, datum, literal digest input in hex)
    (42, 7, "2a" + "00" * 15 + "7c" + "07" + "00" * 15 + "7c"),
    (2**64 - 1, -3, "ff" * 8 + "00" * 8 + "7c" + "fd" + "ff" * 15 + "7c"),
    (5, "rank", "05" + "00" * 15 + "7c" + "72616e6b" + "7c"),
    (0, 0, "00" * 16 + "7c" + "00" * 16 + "7c"),
    (2**40 + 3, 2**33, "03000000" + "0001" + "00" * 10 + "7c" + "00000000" + "02" + "00" * 11 + "7c"),
]


def _blake_le(hexbytes: str) -> int:
    import hashlib

    return int.from_bytes(hashlib.blake2b(bytes.fromhex(hexbytes), digest_size=8).digest(), "little")


@pytest.mark.parametrize("seed,datum,hexbytes", FOLD_IN_KAT)
def test_fold_in_known_answers(seed, datum, hexbytes):
    assert dp_ref.fold_in_seed(seed, datum) == _blake_le(hexbytes)


def test_key_reduces_to_uint64():
    assert dp_ref.key_seed(-1) == 2**64 - 1
    assert dp_ref.key_seed(2**64 + 5) == 5


# ---------------------------------------------------------------------------
# The reference's CPU sampler (dp_ref.gaussian_noise_reference)
# ---------------------------------------------------------------------------


def _ref_uniforms(key: int, step: int, shapes, dtype=torch.float32, stream_fold=None):
    """The generator the reference seeds for (key, step): its seed from the
    fold_in known answers above (fold_in(key, step) mod 2^63 - 1), draws in
    sorted-key order."""
    seed = dp_ref.fold_in_seed(dp_ref.key_seed(key), *(() if stream_fold is None else (stream_fold,)), step)
    gen = torch.Generator().manual_seed(seed % (2**63 - 1))
    return [torch.rand(s, dtype=dtype, generator=gen) for s in shapes]


def test_reference_sampler_statistics():
    """KS, mean and std as the reference's noise tests check them
    (DPS-T/noise/test_noise.py:98-114, test_gaussian_compute_dtype.py:26-39)."""
    from scipy import stats

    out = dp_ref.gaussian_noise_reference({"a": torch.zeros(10_000)}, 1.0, key=42, step=0)["a"].double().numpy()
    assert abs(out.mean()) < 0.05
    assert abs(out.std() - 1.0) < 0.1
    assert stats.kstest(out, "norm").pvalue > 0.01
    bf = dp_ref.gaussian_noise_reference({"a": torch.zeros(16384, dtype=torch.bfloat16)}, 2.0, key=7, step=0)["a"]
    assert bf.dtype == torch.bfloat16 and abs(bf.float().std().item() - 2.0) < 0.05


def test_reference_sampler_determinism_and_passthrough():
    """Same key and step give the same values, another key or step other
    values (test_noise.py:214-259); sigma = 0 returns the input unchanged and
    a bound clamps it (_gaussian.py:245-250)."""
    tree = {"w": torch.randn(50, generator=torch.Generator().manual_seed(0))}
    a = dp_ref.gaussian_noise_reference(tree, 0.5, key=3, step=1)["w"]
    assert torch.equal(a, dp_ref.gaussian_noise_reference(tree, 0.5, key=3, step=1)["w"])
    assert not torch.equal(a, dp_ref.gaussian_noise_reference(tree, 0.5, key=4, step=1)["w"])
    assert not torch.equal(a, dp_ref.gaussian_noise_reference(tree, 0.5, key=3, step=2)["w"])
    assert dp_ref.gaussian_noise_reference(tree, 0.0, key=3, step=1)["w"] is tree["w"]
    clamped = dp_ref.gaussian_noise_reference(tree, 0.0, key=3, step=1, bound=(-0.5, 0.25))["w"]
    assert torch.equal(clamped, tree["w"].clamp(-0.5, 0.25))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_reference_sampler_is_the_inverse_cdf_of_its_stream(dtype):
    """Phi((x - c) / sigma) equals the clamped uniform the generator drew for
    that element, leaf by leaf in sorted-key order, with a sigma = 0 leaf
    drawing nothing; a wrong seed, draw order, sqrt(2) or 2u - 1 fails."""
    from scipy.stats import norm

    g = torch.Generator().manual_seed(1)
    tree = {"z": torch.randn(300, generator=g).to(dtype), "a": torch.randn(4, 5, generator=g).to(dtype),
            "m": torch.randn(7, generator=g).to(dtype)}
    sd = {("a",): 0.7, ("m",): 0.0, ("z",): 1.3}
    out = dp_ref.gaussian_noise_reference(tree, sd, key=11, step=4, compute_dtype=dtype)
    ua, uz = _ref_uniforms(11, 4, [(4, 5), (300,)], dtype)  # "m" draws nothing
    eps = torch.finfo(dtype).eps
    tol = 2e-6 if dtype == torch.float32 else 1e-12
    for name, u, s in (("a", ua, 0.7), ("z", uz, 1.3)):
        got = norm.cdf(((out[name] - tree[name]).double() / s).numpy())
        want = u.clamp(eps, 1 - eps).double().numpy()
        np.testing.assert_allclose(got, want, rtol=0, atol=tol * 8)
    assert out["m"] is tree["m"]


def test_reference_sampler_paired_streams_fold_their_tags():
    """The paired second-moment streams use fold_in(fold_in(key, 1|2), step)
    (_gaussian.py:329-334)."""
    from scipy.stats import norm

    tree = {"g": torch.zeros(64)}
    for fold in (1, 2):
        out = dp_ref.gaussian_noise_reference(tree, 1.0, key=9, step=3, stream_fold=fold)["g"]
        (u,) = _ref_uniforms(9, 3, [(64,)], stream_fold=fold)
        np.testing.assert_allclose(norm.cdf(out.double().numpy()), u.double().numpy(), atol=2e-5)


def test_reference_bounded_sampler_distribution():
    """With bound B and max_norm 1 the output is a truncated normal on
    [-B, B] (DPS-T/noise/test_bounded_gaussian.py:220-235) inside the bound
    (:72-88), with variance below sigma^2 (:237-242)."""
    from scipy import stats

    out = dp_ref.gaussian_noise_reference({"a": torch.zeros(50_000)}, 1.0, key=42, step=0, bound=(-2.0, 2.0))["a"]
    x = out.double().numpy()
    assert x.min() >= -2.0 and x.max() <= 2.0 and x.var() < 1.0
    assert stats.kstest(x, stats.truncnorm.cdf, args=(-2.0, 2.0, 0.0, 1.0)).pvalue > 0.01
    asym = dp_ref.gaussian_noise_reference({"a": torch.zeros(10_000)}, 1.0, key=0, step=0, bound=(-1.0, 4.0))["a"]
    assert asym.min() >= -1.0 and asym.max() <= 4.0


def test_reference_bounded_sampler_reduces_to_the_plain_one():
    """A bound far outside the noise leaves alpha = 0 and beta = 1, so the
    bounded sampler equals the unbounded one on the same stream."""
    tree = {"w": torch.randn(500, generator=torch.Generator().manual_seed(2)).double()}
    a = dp_ref.gaussian_noise_reference(tree, 0.3, key=5, step=1, compute_dtype=torch.float64)["w"]
    b = dp_ref.gaussian_noise_reference(tree, 0.3, key=5, step=1, compute_dtype=torch.float64,
                                        bound=(-1e6, 1e6))["w"]
    torch.testing.assert_close(a, b, rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# The device stream restated (philox_ref): bit layout and transforms
# ---------------------------------------------------------------------------


def test_uniform24_bit_layout_brute_force():
    """Element e's 24-bit uniform is bits [24 (e mod 16), + 24) of the 384-bit
    string of blocks 3 (e >> 4) .. + 2, sliced here from a Python integer."""
    seed, tag, off, n = 0x0123456789ABCDEF, 5, 13, 70
    got = philox_ref.uniform24_for_elements(seed, off, n, tag)
    for i in range(n):
        e = off + i
        big = 0
        for b in range(3):
            ctr = 3 * (e >> 4) + b
            w = philox_ref.philox4x32_10(ctr & 0xFFFFFFFF, ctr >> 32, tag, 0, seed & 0xFFFFFFFF, seed >> 32)
            for q in range(4):
                big |= int(w[q]) << (32 * (4 * b + q))
        assert int(got[i]) == (big >> (24 * (e % 16))) & 0xFFFFFF, i


def test_uniform53_bit_layout_brute_force():
    seed, tag, off, n = 0xFEDCBA9876543210, 2, 7, 9
    got = philox_ref.uniform53_for_elements(seed, off, n, tag)
    for i in range(n):
        e = off + i
        w = philox_ref.philox4x32_10((e >> 1) & 0xFFFFFFFF, e >> 33, tag, 0, seed & 0xFFFFFFFF, seed >> 32)
        pair = int(w[2 * (e & 1)]) | (int(w[2 * (e & 1) + 1]) << 32)
        assert int(got[i]) == pair >> 11


def test_uniform24_is_uniform():
    """Chi-square of the top 8 bits over 2^18 elements, and every value in range."""
    from scipy import stats

    k = philox_ref.uniform24_for_elements(99, 0, 1 << 18)
    assert k.min() >= 0 and k.max() < (1 << 24)
    hist = np.bincount(k >> 16, minlength=256)
    assert stats.chisquare(hist).pvalue > 1e-3


def test_device_stream_transform_is_the_inverse_cdf():
    """Phi of the noise equals the clamped uniform (float32 and float64 grids)."""
    from scipy.stats import norm

    for wide, bits in ((False, 24), (True, 53)):
        x = philox_ref.gaussian_noise(np.zeros(4000), 1.7, seed=77, flat_offset=123, tag=1, wide=wide)
        k = (philox_ref.uniform53_for_elements if wide else philox_ref.uniform24_for_elements)(77, 123, 4000, 1)
        np.testing.assert_allclose(norm.cdf(x / 1.7), philox_ref.uniforms(k, bits), rtol=0, atol=1e-12)


def test_device_stream_bounded_sampler():
    """Truncated normal on the bound; a far bound reduces to the plain sampler;
    sigma = 0 clamps."""
    from scipy import stats

    x = philox_ref.gaussian_noise_bounded(np.zeros(50_000), 1.0, -2.0, 2.0, seed=42)
    assert x.min() >= -2.0 and x.max() <= 2.0
    assert stats.kstest(x, stats.truncnorm.cdf, args=(-2.0, 2.0, 0.0, 1.0)).pvalue > 0.01
    c = np.linspace(-3, 3, 300)
    far = philox_ref.gaussian_noise_bounded(c, 0.4, -1e6, 1e6, seed=8, flat_offset=5)
    np.testing.assert_allclose(far, philox_ref.gaussian_noise(c, 0.4, seed=8, flat_offset=5), atol=1e-9)
    np.testing.assert_array_equal(philox_ref.gaussian_noise_bounded(c, 0.0, -1.0, 2.0, seed=1), np.clip(c, -1, 2))


@pytest.mark.parametrize("wide", [False, True])
def test_device_stream_ks_p_values_are_uniform_over_seeds(wide):
    """A fixed-seed KS test can fail by chance; over many seeds the p-values
    of a sound stream are uniform on [0, 1]."""
    from scipy import stats

    ps = [stats.kstest(philox_ref.gaussian_noise(np.zeros(20_000), 1.0, seed=s, wide=wide), "norm").pvalue
          for s in range(60)]
    assert stats.kstest(ps, "uniform").pvalue > 0.01
