"""Host-side logic of the drop-in API (no GPU): types, per_group, keys, guard, validation."""

from __future__ import annotations

import json
import math
import os

import pytest
import torch

from oracle import dp_ref
from opaque_amd import guard
from opaque_amd.clipping import auto_clipped_grad, clipped_grad, per_group
from opaque_amd.noise import gaussian_noise
from opaque_amd.noise_allocation import paired_noise_stddevs, per_group_noise_stddev
from opaque_amd.pytree import param_path, tree_flatten_with_paths, tree_unflatten
from opaque_amd.random import RngKey, fold_in, key, split, generator_from_key
from opaque_amd.types import ClippedPytree, NoisedPytree, PerGroup, clipped

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "reference_vectors.json")) as _f:
    CASES = {c["name"]: c for c in json.load(_f)["cases"]}


# -- golden values through the product's host code ----------------------------


def test_noise_per_group_sigma_golden():
    case = CASES["noise_per_group_sigma"]
    pg = PerGroup(groups={"w": "small", "b": "large"}, values=case["values"])
    sd = per_group_noise_stddev(pg, case["noise_multiplier"])
    assert sd.values == {k: pytest.approx(v, rel=1e-15) for k, v in case["expected"].items()}
    assert sd.groups == pg.groups


def test_noise_stddev_for_golden():
    case = CASES["noise_stddev_for_scalar"]
    cg = clipped(torch.zeros(8), max_norm=case["max_norm"])
    assert cg.noise_stddev_for(noise_multiplier=case["noise_multiplier"]) == pytest.approx(case["expected"])
    assert cg.noise_stddev_for(noise_multiplier=case["noise_multiplier"], allocation="isotropic") == \
        pytest.approx(case["expected"])


def test_per_group_bound_arithmetic_golden():
    case = CASES["per_group_bound_arithmetic"]
    params = {"a": torch.tensor(1.0), "b": torch.tensor(1.0)}
    pg = per_group(params, **case["patterns"])
    sd = case["noise_multiplier"] * pg
    assert isinstance(sd, PerGroup)
    assert sd.values == {k: pytest.approx(v) for k, v in case["expected"].items()}


def test_per_group_nested_assignment():
    case = CASES["per_group_nested"]
    tree = {k: {kk: torch.tensor(v) for kk, v in d.items()} for k, d in case["tree"].items()}
    pg = per_group(tree, **case["patterns"])
    assert pg.groups[("layer1", "attn")] == "attn"
    assert pg.groups[("layer2", "mlp")] == "mlp"
    assert pg.effective == pytest.approx(math.sqrt(2.0))


def test_per_group_errors():
    params = {"q_proj": torch.zeros(1), "mlp": torch.zeros(1)}
    with pytest.raises(ValueError, match="At least one pattern"):
        per_group(params)
    with pytest.raises(ValueError, match="must be positive"):
        per_group(params, q_proj=0.0, mlp=1.0)
    with pytest.raises(ValueError, match="did not match any pattern"):
        per_group(params, q_proj=1.0)
    with pytest.raises(ValueError, match="matched multiple patterns"):
        per_group(params, q=1.0, q_proj=1.0, mlp=1.0)
    pg = per_group(params, q_proj=1.0, fallback=2.0)
    assert pg.values == {"q_proj": 1.0, "fallback": 2.0}
    with pytest.raises(ValueError, match="Fallback value must be positive"):
        per_group(params, q_proj=1.0, fallback=-1.0)


def test_clipped_pytree_arithmetic():
    c = clipped({"w": torch.ones(2)}, max_norm=2.0)
    assert (c * 3).max_norm == 6.0
    assert (0.5 * c).max_norm == 1.0
    assert (c / 4).max_norm == 0.5
    assert (-c).max_norm == 2.0
    with pytest.raises(TypeError):
        c + c
    with pytest.raises(TypeError):
        c * torch.tensor(2.0)
    with pytest.raises(ZeroDivisionError):
        c / 0
    n = NoisedPytree(pytree={"w": torch.ones(2)}, max_norm=1.0, noise_stddev=0.5)
    assert (2 * n).noise_stddev == 1.0


def test_paired_noise_stddevs_scalar():
    s1, s2 = paired_noise_stddevs(1.5, first=2.0, second=3.0)
    total = 5.0
    assert s1 == pytest.approx(1.5 * math.sqrt(2.0 * total))
    assert s2 == pytest.approx(1.5 * math.sqrt(3.0 * total))


# -- keys and pytree order -----------------------------------------------------


def test_rng_keys_match_oracle():
    k = key(123)
    assert isinstance(k, RngKey)
    for data in [(0,), (7, 3), ("noise",), (2**40, -5)]:
        assert fold_in(k, *data).seed == dp_ref.fold_in_seed(dp_ref.key_seed(123), *data)
    assert fold_in(fold_in(k, 7), 3).seed == fold_in(k, 7, 3).seed
    a, b, c = split(k, 3)
    assert len({a.seed, b.seed, c.seed}) == 3
    assert key(-1).seed == 2**64 - 1


def test_rng_keys_known_answers():
    """fold_in of the product against BLAKE2b digests of literal byte strings
    in the reference's format (ENG/random/_engine.py:27-35: 16-byte
    little-endian signed ints or UTF-8, each followed by b"|")."""
    import hashlib

    def digest(hexbytes):
        return int.from_bytes(hashlib.blake2b(bytes.fromhex(hexbytes), digest_size=8).digest(), "little")

    assert fold_in(key(42), 7).seed == digest("2a" + "00" * 15 + "7c" + "07" + "00" * 15 + "7c")
    assert fold_in(key(-1), -3).seed == digest("ff" * 8 + "00" * 8 + "7c" + "fd" + "ff" * 15 + "7c")
    assert fold_in(key(5), "rank").seed == digest("05" + "00" * 15 + "7c" + "72616e6b" + "7c")
    k = fold_in(key(42), 7)
    assert generator_from_key(k).initial_seed() == k.seed % (2**63 - 1)


def test_pytree_order_sorted_keys_and_roundtrip():
    tree = {"b": torch.zeros(1), "a": [torch.ones(1), {"z": torch.ones(2), "y": None}], "c": (torch.ones(3),)}
    paths, leaves, td = tree_flatten_with_paths(tree)
    assert paths == [("a", 0), ("a", 1, "z"), ("b",), ("c", 0)]
    back = tree_unflatten(td, leaves)
    assert list(back.keys()) == ["b", "a", "c"]
    assert back["a"][1]["y"] is None
    assert param_path("x.y") == ("x.y",)
    assert [p for p, _ in dp_ref.flatten(tree)] == [tuple(p) for p in paths]


# -- guard constants: product host code vs the oracle restatement --------------


@pytest.mark.parametrize("shapes", [[(3,)], [(4096,)], [(4097,), (7, 5)], [(8192, 16), (16, 4096), (1,)]])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_guard_constants_match_oracle(shapes, dt):
    leaves = [torch.zeros(s, dtype=dt) for s in shapes]
    acc, rnd = guard.leaf_guards(shapes, [dt] * len(shapes))
    assert acc == dp_ref.acc_dtype(leaves, None)
    assert rnd == dp_ref.roundoff(acc, len(leaves), dp_ref.reduction_terms(leaves))
    rel, ab = guard.guard_constants(dt, rnd)
    ratio = torch.tensor([0.5, 1.7, 3e-5], dtype=torch.float64)
    expect = dp_ref.finalize(ratio, dt, rnd, clamp_one=False)
    got = torch.clamp(ratio * rel - ab, min=0.0)
    assert torch.equal(got, expect)
    # The magnitude the reference documents (_pytree.py:384-385,492-493): the
    # shrink 1 - rel is one unit roundoff of the storage dtype plus twice the
    # norm roundoff -- neither a smaller nor a larger guard passes.
    eps = torch.finfo(dt).eps
    assert rnd > 0 and abs((1.0 - rel) - eps) <= 2 * rnd * (1 + 1e-9)


# -- validation messages (the reference's tests assert these substrings) --------


def _loss(p, x):
    return (p * x).sum()


@pytest.mark.parametrize(
    "kwargs,exc,match",
    [
        (dict(clipping_norm=1.0, normalize_by=0.0), ValueError, "normalize_by must be > 0"),
        (dict(clipping_norm=1.0, batch_argnums=()), ValueError, "Batch argnums must not be empty"),
        (dict(clipping_norm=1.0, argnums=1, batch_argnums=1), ValueError, "have a batch axis"),
        (dict(clipping_norm=0.0), ValueError, "clipping_norm must be positive"),
        (dict(clipping_norm=1.0, return_aux=True, return_stats=True), ValueError, "return_stats cannot be combined"),
        (dict(clipping_norm=1.0, compute_dtype=torch.int32), TypeError, "compute_dtype"),
    ],
)
def test_clipped_grad_validation(kwargs, exc, match):
    with pytest.raises(exc, match=match):
        clipped_grad(_loss, **kwargs)


def test_clipped_grad_per_group_validation():
    pg = PerGroup(groups={"a": "g"}, values={"g": -1.0})
    with pytest.raises(ValueError, match="clipping_norm must be positive for all groups"):
        clipped_grad(_loss, clipping_norm=pg)


def test_auto_clipped_grad_validation():
    with pytest.raises(ValueError, match="R must be positive"):
        auto_clipped_grad(_loss, R=0.0)
    with pytest.raises(ValueError, match="gamma must be positive"):
        auto_clipped_grad(_loss, gamma=0.0)


def test_product_refuses_cpu_parameters():
    fn, st = clipped_grad(_loss, clipping_norm=1.0)
    with pytest.raises(RuntimeError, match="GPU"):
        fn(torch.ones(3), torch.ones(2, 3), state=st)


def test_outer_differentiating_transform_is_refused():
    """The reference keeps the graph when an enclosing torch.func grad/jvp
    differentiates its clipped gradient (_clipped_grad.py:261-265,
    functional/_transform_stack.py:10-21).  The kernels here are not
    differentiable, so such a call raises a named error before any device
    work; vmap alone and the top level are not differentiating."""
    from opaque_amd.clipping import under_differentiating_transform

    assert not under_differentiating_transform()
    seen = []
    torch.func.vmap(lambda t: seen.append(under_differentiating_transform()) or t)(torch.ones(2))
    torch.func.grad(lambda t: seen.append(under_differentiating_transform()) or t.sum())(torch.ones(2))
    torch.func.jvp(lambda t: seen.append(under_differentiating_transform()) or t, (torch.ones(2),), (torch.ones(2),))
    assert seen == [False, True, True]
    for make in (lambda: clipped_grad(_loss, clipping_norm=1.0),
                 lambda: auto_clipped_grad(_loss, R=1.0)):
        fn, st = make()
        x = torch.ones(3, 4)

        def outer(p):
            return fn(p, x, state=st)[0].pytree.sum()

        with pytest.raises(NotImplementedError, match="not differentiable"):
            torch.func.grad(outer)(torch.ones(4))
        with pytest.raises(NotImplementedError, match="not differentiable"):
            torch.func.jvp(outer, (torch.ones(4),), (torch.ones(4),))


def test_gaussian_noise_validation():
    with pytest.raises(ValueError, match="non-negative"):
        gaussian_noise(noise_multiplier=-1.0, key=key(0))
    with pytest.raises(TypeError, match="RngKey"):
        gaussian_noise(noise_multiplier=1.0, key=0)
    fn, st = gaussian_noise(noise_multiplier=1.0, key=key(0))
    with pytest.raises(TypeError, match="not NoisedPytree"):
        fn(NoisedPytree(pytree=torch.zeros(1), max_norm=1.0, noise_stddev=1.0), st)
    with pytest.raises(TypeError, match="expects ClippedPytree"):
        fn(torch.zeros(1), st)


def test_gaussian_noise_zero_multiplier_passthrough_on_cpu_tree():
    # nm = 0 adds nothing and launches nothing: the same leaf objects come back.
    fn, st = gaussian_noise(noise_multiplier=0.0, key=key(0))
    leaf = torch.ones(8)
    out, st2 = fn(ClippedPytree(leaf, max_norm=float("inf")), st)
    assert out.pytree is leaf and out.noise_stddev == 0.0
    assert st2._step_counter == 1


def test_alias_installs_reference_import_paths():
    import subprocess
    import sys

    code = (
        "import opaque_amd.alias as a; assert a.install();"
        "from opaque.dpsgd.clipping import clipped_grad, auto_clipped_grad, per_group;"
        "from opaque.dpsgd.noise import gaussian_noise;"
        "from opaque.types import ClippedPytree, NoisedPytree, PerGroup;"
        "from opaque.random import key, fold_in;"
        "from opaque.pytree import tree_map;"
        "from opaque.dpsgd.clipping.types import ClippingStats;"
        "import opaque_amd.clipping as c; assert clipped_grad is c.clipped_grad; print('ok')"
    )
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                         cwd=os.path.dirname(HERE))
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "ok"


# -- adaptive clipping: update rule and validation (reference test_adaptive.py:145-218) --


def test_adaptive_update_rule_known_answers():
    from opaque_amd.adaptive import _adaptive_clipping_norm_update as upd

    kw = dict(base_clipping_norm=1.0, target_quantile=0.5, learning_rate=0.2,
              clipping_norm_min=0.01, clipping_norm_max=100.0)
    assert abs(upd(noisy_clipping_rate=0.8, **kw) - math.exp(0.2 * 0.3)) < 1e-6
    assert abs(upd(noisy_clipping_rate=0.2, **kw) - math.exp(-0.2 * 0.3)) < 1e-6
    assert abs(upd(noisy_clipping_rate=0.5, **kw) - 1.0) < 1e-6
    assert upd(noisy_clipping_rate=1e6, **kw) == 100.0
    assert upd(noisy_clipping_rate=-1e6, **kw) == 0.01


def test_adaptive_noisy_rate_is_keyed():
    from opaque_amd.adaptive import _sample_noisy_clipping_rate as noisy

    a = noisy(0.3, key=key(5), step=2, fraction_noise_std=0.05)
    b = noisy(0.3, key=key(5), step=2, fraction_noise_std=0.05)
    c = noisy(0.3, key=key(5), step=3, fraction_noise_std=0.05)
    assert a == b and a != c
    g = torch.Generator().manual_seed(dp_ref.fold_in_seed(dp_ref.key_seed(5), 2) % (2**63 - 1))
    assert a == pytest.approx(0.3 + torch.randn(1, generator=g).item() * 0.05, abs=0)


@pytest.mark.parametrize(
    "kwargs,match",
    [
        (dict(initial_clipping_norm=0.0), "initial_clipping_norm must be positive"),
        (dict(target_quantile=1.0), "target_quantile must be in"),
        (dict(learning_rate=0.0), "learning_rate must be positive"),
        (dict(clipping_norm_min=0.0), "clipping_norm_min must be positive"),
        (dict(clipping_norm_min=1.0, clipping_norm_max=1.0), "must be > clipping_norm_min"),
        (dict(fraction_noise_std=0.0), "fraction_noise_std must be positive"),
        (dict(return_aux=True, return_stats=True), "return_stats cannot be combined"),
    ],
)
def test_adaptive_validation(kwargs, match):
    from opaque_amd.adaptive import adaptive_clipped_grad

    with pytest.raises(ValueError, match=match):
        adaptive_clipped_grad(_loss, key=key(0), **kwargs)


def _helper():
    from opaque_amd import _host

    mod = _host.load()
    if mod is None:
        pytest.skip("host helper not built (opaque_amd.build.build_host)")
    return mod


def _lora_sites(seed=0, share=True, **over):
    from opaque_amd.engine import LoraSite

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(64, 32, generator=g).to(torch.bfloat16)
    sites = []
    for k, d_out in enumerate((48, 16)):
        xs = x if share or k == 0 else x.clone()
        gt = torch.randn(64, d_out, generator=g).to(torch.bfloat16)
        A = torch.randn(32, 8, generator=g).to(torch.bfloat16)
        B = torch.randn(8, d_out, generator=g).to(torch.bfloat16)
        sites.append(LoraSite(xs, gt, A, B, 2.0, a_leaf=2 * k, b_leaf=2 * k + 1))
    for k, v in over.items():
        setattr(sites[1], k, v)
    return sites


def test_host_signature_tracks_structure_and_addresses():
    """The helper's LoRA-site signature (the plan key's LoRA part when the
    helper is built) changes with every field that shapes a plan's tables and
    with nothing else; the addresses it writes are the sites' tensors'."""
    mod = _helper()
    ptrs = torch.empty(12, dtype=torch.int64)
    base = _lora_sites(0)
    sig = mod.lora_signature(base, ptrs)
    assert ptrs.tolist() == [a for s in base for a in (s.x.data_ptr(), s.g.data_ptr(), s.A.data_ptr(),
                                                       s.B.data_ptr(), 0, 0)]
    assert mod.lora_signature(_lora_sites(1), torch.empty(12, dtype=torch.int64)) == sig  # new values, same structure
    # The seam's rank-space products: their presence and layout are structure,
    # their addresses are written beside the others.
    vu = _lora_sites(0)
    for s_ in vu:
        s_.v = (s_.x.float() @ s_.A.float()).to(torch.bfloat16)
        s_.u = (s_.g.float() @ s_.B.float().t()).to(torch.bfloat16)
    sig_vu = mod.lora_signature(vu, ptrs)
    assert sig_vu != sig
    assert ptrs.tolist() == [a for s in vu for a in (s.x.data_ptr(), s.g.data_ptr(), s.A.data_ptr(), s.B.data_ptr(),
                                                     s.v.data_ptr(), s.u.data_ptr())]
    vu[1].u = vu[1].u.t().contiguous().t()
    assert mod.lora_signature(vu, torch.empty(12, dtype=torch.int64)) != sig_vu
    g_t = base[1].g.t().contiguous().t()  # same shape, other strides
    changed = {
        "unshared x": _lora_sites(0, share=False),
        "g strides": _lora_sites(0, g=g_t),
        "g dtype": _lora_sites(0, g=base[1].g.float()),
        "g shape": _lora_sites(0, g=base[1].g[:32]),
        "g alignment": _lora_sites(0, g=torch.empty(64 * 16 + 1, dtype=torch.bfloat16)[1:].view(64, 16)),
        "A shape": _lora_sites(0, A=base[1].A[:, :4]),
        "B non-contiguous": _lora_sites(0, B=base[1].B.t().contiguous().t()),
        "B dtype": _lora_sites(0, B=base[1].B.float()),
        "scaling": _lora_sites(0, scaling=4.0),
        "a_leaf": _lora_sites(0, a_leaf=None),
        "b_transposed": _lora_sites(0, b_transposed=True),
    }
    for what, sites in changed.items():
        assert mod.lora_signature(sites, torch.empty(12, dtype=torch.int64)) != sig, what
    from opaque_amd.engine import Segments

    assert mod.lora_signature(_lora_sites(0, segments=Segments.padded(2, 32)), ptrs) is None


def test_host_view_maker_matches_torch_views():
    mod = _helper()
    a = torch.arange(200, dtype=torch.float32)
    b = torch.arange(100, dtype=torch.bfloat16)
    vm = mod.ViewMaker([0, 1, 0], [[3, 4], [10], []], [[4, 1], [1], []], [64, 0, 7])
    v = vm.make([a, b])
    assert torch.equal(v[0], a[64:76].view(3, 4)) and v[0].data_ptr() == a.data_ptr() + 64 * 4
    assert torch.equal(v[1], b[:10]) and v[2].shape == () and v[2].item() == 7.0
    # views of other dtypes over a byte buffer (offsets count the view's elements)
    raw = torch.arange(1024, dtype=torch.int32).view(torch.uint8)
    vm2 = mod.ViewMaker([0, 0], [[2, 3], [4]], [[3, 1], [1]], [32, 512],
                        [torch.empty(0, dtype=torch.float64), torch.empty(0, dtype=torch.uint8)])
    d, u = vm2.make([raw])
    assert d.dtype == torch.float64 and torch.equal(d, raw[256 : 256 + 48].view(torch.float64).view(2, 3))
    assert u.dtype == torch.uint8 and torch.equal(u, raw[512:516])


@pytest.mark.parametrize("avail_gib", [0, 1, 6, 40, 200, 288])
@pytest.mark.parametrize("stored_frac", [0.0, 0.5])
def test_plan_memory_budgets_fit_the_device(avail_gib, stored_frac):
    """Stored per-example gradients (at most half the available memory by
    default), the Gram scratch and the prescaled activations come out of one
    reading of the available memory and never add up to more than it."""
    from opaque_amd.engine import GRAM256_SCRATCH_BYTES, split_budget

    avail = avail_gib << 30
    stored = int(avail * stored_frac) // 2 * 2
    scr, pre = split_budget(avail, stored, 8 << 30)
    assert 0 <= scr <= GRAM256_SCRATCH_BYTES and 0 <= pre <= 8 << 30
    assert stored + scr + pre <= avail
    if avail_gib == 288 and stored_frac == 0.0:
        assert (scr, pre) == (GRAM256_SCRATCH_BYTES, 8 << 30)  # a whole MI355X: both at their caps
    # The budgets shrink with what is left: a caller holding most of the
    # device leaves less to each.
    if avail_gib:
        scr2, pre2 = split_budget(avail // 4, stored // 4, 8 << 30)
        assert scr2 <= scr and pre2 <= pre
    assert split_budget(None, 0, 123) == (GRAM256_SCRATCH_BYTES, 123)  # off the GPU: no device limit


def test_form_choice_at_c4_shapes():
    """At 4096 tokens the 256-row-block Gram kernel makes the token-Gram norm
    the cheaper form for gate/up/down (L (d_in + d_out) below d_in d_out at
    its measured cost per flop); q/o and k/v stay with the outer form, and
    short segments use the 128-row-block cost."""
    from opaque_amd import _native as N
    from opaque_amd.engine import choose_form

    assert choose_form(4096, 4096, 14336) == N.FORM_GRAM
    assert choose_form(4096, 14336, 4096) == N.FORM_GRAM
    assert choose_form(4096, 4096, 4096) == N.FORM_OUTER
    assert choose_form(4096, 4096, 1024) == N.FORM_OUTER
    assert choose_form(64, 512, 512) == N.FORM_GRAM
    assert choose_form(500, 700, 700) == N.FORM_OUTER  # 1.6 * 500 * 1400 > 2 * 700 * 700
