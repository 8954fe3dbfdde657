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
