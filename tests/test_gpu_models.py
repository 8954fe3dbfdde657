"""End to end on a real model: a random-init Hugging Face Llama (GQA attention,
RMSNorm, SwiGLU, rotary embeddings, cross-entropy) with LoRA adapters injected
through the seam (``capture.inject_lora``), clipped by the drop-in
``clipped_grad`` / ``auto_clipped_grad`` on the GPU and by the CPU oracle
(vmap(grad) + the reference's clip + fp32 sum) on a float32 copy.

Tolerances: float32 rel <= 1e-5; bfloat16 rel <= 2e-2.  In bfloat16 the
oracle differentiates the bfloat16 model on the CPU, so both sides round the
forward the same way up to kernel-order effects.
"""

from __future__ import annotations

import copy

import pytest
import torch

from oracle import dp_ref
from opaque_amd import capture
from opaque_amd.clipping import auto_clipped_grad, clipped_grad

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")
DEV = "cuda"


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.norm().item()
    return (a - b).norm().item() / den if den > 0 else (a - b).norm().item()


def _llama(dtype, seed=0, hidden=64, inter=96, layers=2, r=8):
    torch.manual_seed(seed)
    cfg = transformers.LlamaConfig(vocab_size=128, hidden_size=hidden, intermediate_size=inter,
                                   num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                                   max_position_embeddings=128, attn_implementation="eager")
    m = transformers.LlamaForCausalLM(cfg).eval()
    names = capture.inject_lora(m, r=r, alpha=2 * r)
    for mod in m.modules():
        if isinstance(mod, capture.LoRALinear):
            torch.nn.init.normal_(mod.lora_B, std=0.05)
    return m.to(dtype), names


def _loss(m):
    def split(params):
        return {k: v for k, v in m.named_parameters() if k not in params}

    def loss_fn(params, ids, labels):
        out = torch.func.functional_call(m, {**split(params), **params}, (ids.unsqueeze(0),),
                                         {"labels": labels.unsqueeze(0)})
        return out.loss

    return loss_fn


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("autos", [False, True])
def test_hf_llama_lora_matches_oracle(dtype, tol, autos):
    print(f"hf llama: dtype={dtype} autos={autos}", flush=True)
    m_cpu, names = _llama(dtype)
    m_gpu = copy.deepcopy(m_cpu).to(DEV)
    train_cpu = {k: v for k, v in m_cpu.named_parameters() if v.requires_grad}
    train_gpu = {k: v for k, v in m_gpu.named_parameters() if v.requires_grad}
    assert len(train_gpu) == 2 * len(names) == 28
    n, T = 6, 24
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 128, (n, T), generator=g)
    labels = torch.randint(0, 128, (n, T), generator=g)
    ref_loss = _loss(m_cpu)
    _, aux0 = dp_ref.clipped_grad(ref_loss, train_cpu, (ids, labels), clipping_norm=float("inf"))
    C = float(aux0["norms"].detach().median())  # about half the examples clip
    if autos:
        fn, st = auto_clipped_grad(_loss(m_gpu), R=C, batch_argnums=(1, 2), return_aux=True, normalize_by=n)
    else:
        fn, st = clipped_grad(_loss(m_gpu), clipping_norm=C, batch_argnums=(1, 2), return_aux=True,
                              normalize_by=n)
    (grads, gaux), _ = fn(train_gpu, ids.to(DEV), labels.to(DEV), state=st)
    torch.cuda.synchronize()
    disc = fn.engine._discovery[1]
    assert len(disc.eligible) == 28  # every adapter factor went through the seam
    # The seams kept V = x A and U = g B^T: the step reads them instead of
    # projecting the activations and output gradients again.
    live = {t[0] for t in fn.engine._plan.tables if t[5] > 0}
    assert "planes" in live and not live & {"project", "factor_project"}, live
    summed, aux = dp_ref.clipped_grad(ref_loss, train_cpu, (ids, labels), clipping_norm=C, autos=autos,
                                      normalize_by=n)
    for k, ref in summed.items():
        got = grads.pytree[k]
        assert got.dtype == dtype and got.shape == ref.shape, k
        assert rel(got, ref) <= tol, (k, rel(got, ref))
    assert rel(gaux.grad_norms, aux["norms"]) <= tol
    assert rel(gaux.loss_values, aux["loss_values"]) <= tol


class _MoEBlock(torch.nn.Module):
    """Pre-norm residual MoE block (softmax top-2 router, stacked expert weights)."""

    def __init__(self, H=64, inter=32, E=4, K=2):
        super().__init__()
        self.k = K
        self.norm = torch.nn.LayerNorm(H)
        self.router = torch.nn.Linear(H, E, bias=False)
        self.gate_up_proj = torch.nn.Parameter(torch.randn(E, 2 * inter, H) * H**-0.5)
        self.down_proj = torch.nn.Parameter(torch.randn(E, H, inter) * inter**-0.5)

    def forward(self, x):
        h = self.norm(x)
        w, idx = torch.topk(self.router(h).float().softmax(-1), self.k, dim=-1)
        w = (w / w.sum(-1, keepdim=True)).to(x.dtype)
        return x + capture.moe(h, self.gate_up_proj, self.down_proj, idx, w)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_moe_block_matches_oracle(dtype, tol):
    """Expert weights clipped per (example, expert) segment; router and norm by per-example autograd."""
    print(f"moe block: dtype={dtype}", flush=True)
    torch.manual_seed(3)
    m_cpu = _MoEBlock().to(dtype)
    m_gpu = copy.deepcopy(m_cpu).to(DEV)
    train_cpu = dict(m_cpu.named_parameters())
    train_gpu = dict(m_gpu.named_parameters())
    n, T = 6, 24
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(n, T, 64, generator=g) * torch.logspace(-0.5, 0.5, n).view(n, 1, 1)).to(dtype)
    y = torch.randn(n, T, 64, generator=g).to(dtype)

    def loss_of(m):
        def loss_fn(params, xb, yb):
            return ((torch.func.functional_call(m, params, (xb,)).float() - yb.float()) ** 2).mean()
        return loss_fn

    _, aux0 = dp_ref.clipped_grad(loss_of(m_cpu), train_cpu, (x, y), clipping_norm=float("inf"))
    C = float(aux0["norms"].detach().median())
    fn, st = clipped_grad(loss_of(m_gpu), clipping_norm=C, batch_argnums=(1, 2), return_aux=True)
    (grads, gaux), _ = fn(train_gpu, x.to(DEV), y.to(DEV), state=st)
    torch.cuda.synchronize()
    disc = fn.engine._discovery[1]
    assert len(disc.eligible) == 2  # the two stacked expert weights went through the seam
    summed, aux = dp_ref.clipped_grad(loss_of(m_cpu), train_cpu, (x, y), clipping_norm=C)
    for k, ref in summed.items():
        got = grads.pytree[k]
        assert got.dtype == dtype and got.shape == ref.shape, k
        assert rel(got, ref) <= tol, (k, rel(got, ref))
    assert rel(gaux.grad_norms, aux["norms"]) <= tol
