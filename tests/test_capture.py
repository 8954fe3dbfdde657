"""Seam capture on the CPU: discovery, the batched capture pass and what it records.

The per-example factor gradients rebuilt from the recorded (x, g) pairs
(dA_i = s X_i^T G_i B^T, dB_i = s (X_i A)^T G_i) must equal torch.func's
vmap(grad) of the same loss; non-captured leaves get theirs from the
batch-expanded copies.  No kernel runs here.
"""

from __future__ import annotations

import torch

from opaque_amd import capture
from opaque_amd import clipping as C
from opaque_amd.pytree import tree_flatten_with_paths, tree_unflatten


class _Model(torch.nn.Module):
    def __init__(self, bias: bool = True) -> None:
        super().__init__()
        self.q = capture.LoRALinear(16, 24, 4, alpha=8)
        self.o = capture.LoRALinear(24, 16, 4, alpha=8, bias=bias)
        self.ln = torch.nn.LayerNorm(24)
        torch.nn.init.normal_(self.q.lora_B, std=0.1)
        torch.nn.init.normal_(self.o.lora_B, std=0.1)

    def forward(self, x):
        return self.o(torch.tanh(self.ln(self.q(x))))


def _engine(loss_fn, batch_argnums=(1, 2)):
    return C._ClipEngine(
        loss_fn, (0,), 0, False, clipping_norm=1.0, autos=False, gamma=0.0, normalize_by=1.0,
        batch_argnums=batch_argnums, want_aux=False, want_stats=False, second_moment=False,
        pre_clipping_transform=C._identity, microbatch_size=None, dtype=None, compute_dtype=None,
        scale_fn=None,
    )


def _capture_per_example(eng, args, n):
    """The capture pass of the engine, returning per-example grads by leaf path."""
    paths, leaves, td = tree_flatten_with_paths(eng._grad_tree(args))
    disc = eng._discover(args, {}, leaves, td)
    expanded, passed, dims = {}, [], []
    for k, t in enumerate(leaves):
        if k in disc.eligible:
            passed.append(t)
            dims.append(None)
        else:
            e = t.detach().unsqueeze(0).expand(n, *t.shape).requires_grad_()
            expanded[k] = e
            passed.append(e)
            dims.append(0)
    cargs = eng._with_grad_tree(args, tree_unflatten(td, passed))
    in_dims = eng._in_dims(cargs, tree_unflatten(td, dims))
    anchor = torch.zeros((), requires_grad=True)
    obj_leaf = {id(leaves[k]): k for k in disc.eligible}
    sess = capture.CaptureSession(mode="capture", anchor=anchor, eligible=set(obj_leaf))
    with torch.enable_grad(), sess:
        values, _ = torch.func.vmap(lambda *a: eng._loss(*a), in_dims=in_dims, randomness="same")(*cargs)
    grads = torch.autograd.grad(values.sum(), [anchor] + [expanded[k] for k in sorted(expanded)],
                                allow_unused=True)
    got = {paths[k]: g for k, g in zip(sorted(expanded), grads[1:])}
    for r in sess.sites:
        if r.segments is not None:  # an MoE expert's slice of a stacked weight
            k = obj_leaf[id(r.w_obj)]
            pe = C._expert_per_example(r, leaves[k], n)
            got[paths[k]] = got[paths[k]] + pe if paths[k] in got else pe
            continue
        if r.w_obj is not None:
            found = C._site_per_example(r, None, None, leaves, obj_leaf[id(r.w_obj)])
        else:
            ka, kb = obj_leaf.get(id(r.a_obj)), obj_leaf.get(id(r.b_obj))
            found = C._site_per_example(r, ka, kb, leaves)
        for k, pe in found:
            got[paths[k]] = pe
    return disc, sess, got, paths


def _check(ref, got):
    rp, rl, _ = tree_flatten_with_paths(ref)
    assert set(got) == set(rp)
    for p, t in zip(rp, rl):
        torch.testing.assert_close(got[p], t, rtol=1e-5, atol=1e-6)


def test_capture_reproduces_vmap_grad():
    torch.manual_seed(0)
    m = _Model()
    train = {k: v for k, v in m.named_parameters() if v.requires_grad}
    train["ln.weight"] = m.ln.weight
    frozen = {k: v for k, v in m.named_parameters() if k not in train}

    def loss_fn(params, x, y):
        out = torch.func.functional_call(m, {**frozen, **params}, (x,))
        return ((out - y) ** 2).mean()

    n = 3
    x, y = torch.randn(n, 5, 16), torch.randn(n, 5, 16)
    ref = torch.func.vmap(torch.func.grad(loss_fn), in_dims=(None, 0, 0))(train, x, y)
    eng = _engine(loss_fn)
    disc, sess, got, paths = _capture_per_example(eng, (train, x, y), n)
    eligible = {paths[k][0] for k in disc.eligible}
    assert eligible == {"q.lora_A", "q.lora_B", "o.lora_A", "o.lora_B"}
    assert len(sess.sites) == 2
    assert all(r.g is not None and r.x.shape[0] == n for r in sess.sites)
    _check(ref, got)


def test_trainable_bias_and_base_weight():
    torch.manual_seed(1)
    m = _Model(bias=True)
    # The o-projection's bias is trainable (a per-example leaf through the seam's
    # batched bias path); the q-projection's base weight is trainable, which
    # keeps its whole seam off the capture route.
    train = {k: v for k, v in m.named_parameters() if "lora" in k}
    train["o.bias"] = m.o.bias
    train["q.weight"] = m.q.weight
    frozen = {k: v for k, v in m.named_parameters() if k not in train}

    def loss_fn(params, x, y):
        out = torch.func.functional_call(m, {**frozen, **params}, (x,))
        return ((out - y) ** 2).sum()

    n = 4
    x, y = torch.randn(n, 3, 16), torch.randn(n, 3, 16)
    ref = torch.func.vmap(torch.func.grad(loss_fn), in_dims=(None, 0, 0))(train, x, y)
    disc, sess, got, paths = _capture_per_example(_engine(loss_fn), (train, x, y), n)
    assert {paths[k][0] for k in disc.eligible} == {"o.lora_A", "o.lora_B"}
    _check(ref, got)


def test_factor_used_outside_the_seam_is_not_captured():
    g = torch.Generator().manual_seed(2)
    W = torch.randn(8, 8, generator=g)
    params = {"A": torch.randn(8, 2, generator=g), "B": torch.randn(2, 8, generator=g)}

    def loss_fn(p, x):
        y = capture.lora_linear(x, W, p["A"], p["B"], 0.5)
        return (y**2).sum() + (p["A"] ** 2).sum() * x.sum()

    x = torch.randn(3, 8, generator=g)
    ref = torch.func.vmap(torch.func.grad(loss_fn), in_dims=(None, 0))(params, x)
    disc, sess, got, paths = _capture_per_example(_engine(loss_fn, batch_argnums=(1,)), (params, x), 3)
    assert disc.eligible == frozenset()
    assert sess.sites == []
    _check(ref, got)


def test_seam_ops_are_plain_math_outside_capture():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 5, 8, generator=g)
    W = torch.randn(6, 8, generator=g)
    a_w = torch.randn(3, 8, generator=g)
    b_w = torch.randn(6, 3, generator=g)
    bias = torch.randn(6, generator=g)
    y = capture.peft_lora_linear(x, W, a_w, b_w, 1.5, bias)
    torch.testing.assert_close(y, x @ W.t() + bias + 1.5 * (x @ a_w.t()) @ b_w.t())
    y2 = capture.lora_linear(x, W, a_w.t(), b_w.t(), 1.5)
    torch.testing.assert_close(y2, x @ W.t() + 1.5 * (x @ a_w.t()) @ b_w.t())


def test_nested_sessions_rejected():
    import pytest

    with capture.CaptureSession(mode="discover"):
        with pytest.raises(RuntimeError, match="nested"):
            with capture.CaptureSession(mode="discover"):
                pass
    assert capture.active_session() is None


def test_full_weight_linear_seams():
    torch.manual_seed(4)

    class Net(torch.nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.a = capture.Linear(12, 20, bias=True)
            self.b = capture.Linear(20, 12, bias=False)
            self.shared = capture.Linear(12, 12, bias=False)

        def forward(self, x):
            h = torch.relu(self.a(x))
            y = self.b(h)
            # `shared` is applied twice: two seam uses, so it is not captured.
            return self.shared(self.shared(y))

    net = Net()
    params = dict(net.named_parameters())

    def loss_fn(p, x, y):
        return ((torch.func.functional_call(net, p, (x,)) - y) ** 2).mean()

    n = 3
    x, y = torch.randn(n, 4, 12), torch.randn(n, 4, 12)
    ref = torch.func.vmap(torch.func.grad(loss_fn), in_dims=(None, 0, 0))(params, x, y)
    disc, sess, got, paths = _capture_per_example(_engine(loss_fn), (params, x, y), n)
    assert {paths[k][0] for k in disc.eligible} == {"a.weight", "b.weight"}
    assert sorted(r.kind for r in sess.sites) == ["linear", "linear"]
    _check(ref, got)


def _tiny_llama(seed=0, dtype=torch.float32):
    """A random-init two-layer Llama (GQA attention, RMSNorm, SwiGLU) with LoRA on all seven projections."""
    transformers = __import__("pytest").importorskip("transformers")
    torch.manual_seed(seed)
    cfg = transformers.LlamaConfig(vocab_size=64, hidden_size=32, intermediate_size=48, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
                                   attn_implementation="eager")
    m = transformers.LlamaForCausalLM(cfg).to(dtype).eval()
    names = capture.inject_lora(m, r=4, alpha=8)
    for mod in m.modules():
        if isinstance(mod, capture.LoRALinear):
            torch.nn.init.normal_(mod.lora_B, std=0.1)
    return m, names


def test_inject_lora_on_hf_llama_reproduces_vmap_grad():
    m, names = _tiny_llama()
    assert len(names) == 14
    train = {k: v for k, v in m.named_parameters() if v.requires_grad}
    assert set(train) == {f"{n}.{f}" for n in names for f in ("lora_A", "lora_B")}
    frozen = {k: v for k, v in m.named_parameters() if k not in train}

    def loss_fn(params, ids, labels):
        out = torch.func.functional_call(m, {**frozen, **params}, (ids.unsqueeze(0),),
                                         {"labels": labels.unsqueeze(0)})
        return out.loss

    n, T = 3, 8
    g = torch.Generator().manual_seed(1)
    ids, labels = torch.randint(0, 64, (n, T), generator=g), torch.randint(0, 64, (n, T), generator=g)
    ref = torch.func.vmap(torch.func.grad(loss_fn), in_dims=(None, 0, 0), randomness="same")(train, ids, labels)
    eng = _engine(loss_fn)
    disc, sess, got, paths = _capture_per_example(eng, (train, ids, labels), n)
    assert len(disc.eligible) == 28 and len(sess.sites) == 14
    _check(ref, got)


def test_route_linears_reproduces_vmap_grad():
    m, _ = _tiny_llama(seed=2)
    for p in m.parameters():
        p.requires_grad_(False)
    for mod in m.modules():  # drop the adapters' trainability; train two full weights instead
        if isinstance(mod, capture.LoRALinear):
            mod.lora_A.requires_grad_(False)
            mod.lora_B.requires_grad_(False)
    lm = m.lm_head
    routed = capture.route_linears(m, ("lm_head",))
    assert routed == ["lm_head"] and m.lm_head.weight is lm.weight
    m.lm_head.weight.requires_grad_(True)
    train = {k: v for k, v in m.named_parameters() if v.requires_grad}
    frozen = {k: v for k, v in m.named_parameters() if k not in train}

    def loss_fn(params, ids, labels):
        out = torch.func.functional_call(m, {**frozen, **params}, (ids.unsqueeze(0),),
                                         {"labels": labels.unsqueeze(0)})
        return out.loss

    n, T = 2, 6
    g = torch.Generator().manual_seed(3)
    ids, labels = torch.randint(0, 64, (n, T), generator=g), torch.randint(0, 64, (n, T), generator=g)
    ref = torch.func.vmap(torch.func.grad(loss_fn), in_dims=(None, 0, 0), randomness="same")(train, ids, labels)
    eng = _engine(loss_fn)
    disc, sess, got, paths = _capture_per_example(eng, (train, ids, labels), n)
    assert len(disc.eligible) == 1
    _check(ref, got)


class _MoEBlock(torch.nn.Module):
    """Pre-norm residual MoE block: softmax top-k router, stacked expert weights."""

    def __init__(self, H=16, inter=8, E=4, K=2):
        super().__init__()
        self.k = K
        self.norm = torch.nn.LayerNorm(H)
        self.router = torch.nn.Linear(H, E, bias=False)
        self.gate_up_proj = torch.nn.Parameter(torch.randn(E, 2 * inter, H) * H**-0.5)
        self.down_proj = torch.nn.Parameter(torch.randn(E, H, inter) * inter**-0.5)

    def forward(self, x):
        h = self.norm(x)
        w, idx = torch.topk(self.router(h).softmax(-1), self.k, dim=-1)
        w = w / w.sum(-1, keepdim=True)
        return x + capture.moe(h, self.gate_up_proj, self.down_proj, idx, w)


def test_moe_experts_reproduce_vmap_grad():
    torch.manual_seed(4)
    m = _MoEBlock()
    train = dict(m.named_parameters())  # experts captured; router and norm per-example by autograd

    def loss_fn(params, x, y):
        return ((torch.func.functional_call(m, params, (x,)) - y) ** 2).mean()

    n, T = 3, 7
    x, y = torch.randn(n, T, 16), torch.randn(n, T, 16)
    ref = torch.func.vmap(torch.func.grad(loss_fn), in_dims=(None, 0, 0))(train, x, y)
    eng = _engine(loss_fn)
    disc, sess, got, paths = _capture_per_example(eng, (train, x, y), n)
    assert {paths[k][0] for k in disc.eligible} == {"gate_up_proj", "down_proj"}
    assert len(sess.sites) == 2 * 4 and all(r.segments is not None for r in sess.sites)
    # Each expert's rows: one segment per example, lengths summing to the routed tokens.
    assert sum(sum(r.segments.lengths) for r in sess.sites[::2]) == n * T * 2
    _check(ref, got)
