"""Capture of (activation, output-gradient) pairs at LoRA seams.

The reference computes per-example LoRA gradients inside the ``vmap`` rule of
its LoRA autograd Functions (``opaque-patches/.../kernels/lora.py:145-184``,
fed by ``PAT/peft/components/linear.py:60-68``).  Here the same seam records
what the DP kernels need instead: the activations ``x`` of the whole batch
and, during one ordinary backward pass, the output gradients ``g``.  The
per-example factor gradients are then never materialised by autograd.

Outside a capture pass the ops are plain differentiable torch math
(``y = x W^T + s (x A) B``), so the same model code runs under the
reference's ``vmap(grad)``, under ordinary autograd and under the engine.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass, field
from typing import Any

import torch
import torch.nn.functional as F

_STATE = threading.local()


@dataclass
class SiteRecord:
    """One LoRA (or full-weight linear) application seen during a capture pass."""

    x: torch.Tensor  # physical activations [B, *, d_in]
    A: torch.Tensor | None  # kernel-layout [d_in, r] values (LoRA)
    B: torch.Tensor | None  # kernel-layout [r, d_out] values (LoRA)
    scaling: float
    a_obj: torch.Tensor | None  # the tensor the model passed (identity used for leaf lookup)
    b_obj: torch.Tensor | None
    a_transposed: bool
    b_transposed: bool
    g: torch.Tensor | None = None  # physical output gradients, filled by backward
    w_obj: torch.Tensor | None = None  # full-weight linear: the weight passed ([d_out, d_in])
    w_index: int | None = None  # MoE expert: slice of the stacked weight w_obj ([E, d_out, d_in])
    segments: Any = None  # MoE expert: engine Segments of x's rows (x is then [rows, d_in])
    v: torch.Tensor | None = None  # LoRA: x A, kept from the forward ([B, *, r])
    u: torch.Tensor | None = None  # LoRA: g B^T, kept from the backward ([B, *, r])

    @property
    def kind(self) -> str:
        return "linear" if self.w_obj is not None else "lora"


@dataclass
class CaptureSession:
    """Active while the engine runs a loss function to capture its LoRA seams.

    ``mode`` is "discover" (record which tensors feed LoRA seams, keep them out
    of autograd) or "capture" (record x and, in backward, g).
    """

    mode: str
    anchor: torch.Tensor | None = None
    sites: list[SiteRecord] = field(default_factory=list)
    uses: dict[int, int] = field(default_factory=dict)  # id(tensor) -> number of seam uses
    pairs: list[tuple[int, int, int, int]] = field(default_factory=list)  # ids of (A, B, W, bias) per call
    linear_ws: list[int] = field(default_factory=list)  # ids of weights of full-weight linear seams
    eligible: set[int] = field(default_factory=set)  # ids allowed to be captured

    def __enter__(self) -> CaptureSession:
        if getattr(_STATE, "session", None) is not None:
            raise RuntimeError("nested opaque_amd capture sessions are not supported")
        _STATE.session = self
        return self

    def __exit__(self, *exc: Any) -> None:
        _STATE.session = None


def active_session() -> CaptureSession | None:
    return getattr(_STATE, "session", None)


def _plain(x, W, A, B, scaling, bias):
    out = F.linear(x, W) + scaling * ((x @ A) @ B)
    return out if bias is None else out + bias


class _TapLoRA(torch.autograd.Function):
    """Physical (batch-merged) LoRA op that records x now and g in backward,
    and with them the rank-space products the op computes anyway: v = x A
    in the forward, u = g B^T in the backward (the reference's merged dX
    forms the same grad_out @ B.t(), PAT/kernels/lora.py:157-160)."""

    @staticmethod
    def forward(x, W, A, B, scaling, bias, anchor, record):
        xa = x @ A
        record.v = xa
        out = F.linear(x, W) + scaling * (xa @ B)
        return out if bias is None else out + bias

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, W, A, B, scaling, bias, anchor, record = inputs
        ctx.save_for_backward(W, A, B)
        ctx.scaling = scaling
        ctx.record = record
        ctx.has_bias = bias is not None
        ctx.bias_batched = bias is not None and bias.dim() > 1

    @staticmethod
    def backward(ctx, g):
        W, A, B = ctx.saved_tensors
        ctx.record.g = g.detach()
        gb = g @ B.t()
        ctx.record.u = gb.detach()
        dx = None
        if ctx.needs_input_grad[0]:
            dx = g @ W + ctx.scaling * (gb @ A.t())
        dbias = None
        if ctx.has_bias and ctx.needs_input_grad[5]:
            # A batched (per-example, [B, 1.., d_out]) bias keeps its example axis.
            if ctx.bias_batched:
                red = tuple(range(1, g.dim() - 1))
                dbias = g.sum(dim=red, keepdim=True) if red else g
            else:
                dbias = g.reshape(-1, g.shape[-1]).sum(0)
        danchor = torch.zeros((), dtype=g.dtype, device=g.device) if ctx.needs_input_grad[6] else None
        return dx, None, None, None, None, dbias, danchor, None


class _SeamLoRA(torch.autograd.Function):
    """Per-example LoRA op whose vmap rule merges the batch and taps the seam."""

    generate_vmap_rule = False

    @staticmethod
    def forward(x, W, A, B, scaling, bias, a_obj, b_obj, a_t, b_t):
        return _plain(x, W, A, B, scaling, bias)

    @staticmethod
    def setup_context(ctx, inputs, output):
        pass

    @staticmethod
    def backward(ctx, g):
        raise RuntimeError("the capture seam is differentiated through its vmap rule only")

    @staticmethod
    def vmap(info, in_dims, x, W, A, B, scaling, bias, a_obj, b_obj, a_t, b_t):
        sess = active_session()
        xd, wd, ad, bd = in_dims[0], in_dims[1], in_dims[2], in_dims[3]
        bias_d = in_dims[5]
        if xd is None:
            x = x.unsqueeze(0).expand(info.batch_size, *x.shape)
        elif xd != 0:
            x = x.movedim(xd, 0)
        if bias is not None and bias_d is not None and bias_d != 0:
            bias = bias.movedim(bias_d, 0)
        if wd is not None or ad is not None or bd is not None or sess is None or sess.mode != "capture":
            # A batched (expanded) weight or no capture: plain batched math.
            if wd is not None:
                W = W.movedim(wd, 0)
                out = torch.einsum("b...i,boi->b...o", x, W)
            else:
                out = F.linear(x, W)
            Ab = A.movedim(ad, 0) if ad is not None else A
            Bb = B.movedim(bd, 0) if bd is not None else B
            xa = torch.einsum("b...i,bir->b...r", x, Ab) if ad is not None else x @ Ab
            xab = torch.einsum("b...r,bro->b...o", xa, Bb) if bd is not None else xa @ Bb
            out = out + scaling * xab
            if bias is not None:
                out = out + (bias.view(bias.shape[0], *([1] * (out.dim() - 2)), bias.shape[-1])
                             if bias_d is not None else bias)
            return out, 0
        rec = SiteRecord(x=x, A=A, B=B, scaling=float(scaling), a_obj=a_obj, b_obj=b_obj,
                         a_transposed=a_t, b_transposed=b_t)
        sess.sites.append(rec)
        if bias is not None and bias_d is not None:
            bias = bias.view(bias.shape[0], *([1] * (x.dim() - 2)), bias.shape[-1])
        out = _TapLoRA.apply(x, W, A, B, float(scaling), bias, sess.anchor, rec)
        return out, 0


def _lora(x, W, A, B, scaling, bias, a_obj, b_obj, a_t, b_t):
    sess = active_session()
    if sess is None:
        return _plain(x, W, A, B, scaling, bias)
    if sess.mode == "discover":
        for t in (a_obj, b_obj):
            if t is not None:
                sess.uses[id(t)] = sess.uses.get(id(t), 0) + 1
        sess.pairs.append((id(a_obj), id(b_obj), id(W), id(bias) if bias is not None else 0))
        # Seam parameters are hidden from autograd here, so a gradient that still
        # reaches them afterwards reveals a use outside a seam.
        return _plain(x, W, A.detach(), B.detach(), scaling, bias)
    if id(a_obj) not in sess.eligible and id(b_obj) not in sess.eligible:
        return _plain(x, W, A, B, scaling, bias)
    return _SeamLoRA.apply(x, W, A, B, scaling, bias, a_obj, b_obj, a_t, b_t)


class _TapLinear(torch.autograd.Function):
    """Physical full-weight linear that records x now and g in backward."""

    @staticmethod
    def forward(x, W, bias, anchor, record):
        return F.linear(x, W) if bias is None else F.linear(x, W) + bias

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, W, bias, anchor, record = inputs
        ctx.save_for_backward(W)
        ctx.record = record
        ctx.has_bias = bias is not None
        ctx.bias_batched = bias is not None and bias.dim() > 1

    @staticmethod
    def backward(ctx, g):
        (W,) = ctx.saved_tensors
        ctx.record.g = g.detach()
        dx = g @ W if ctx.needs_input_grad[0] else None
        dbias = None
        if ctx.has_bias and ctx.needs_input_grad[2]:
            if ctx.bias_batched:
                red = tuple(range(1, g.dim() - 1))
                dbias = g.sum(dim=red, keepdim=True) if red else g
            else:
                dbias = g.reshape(-1, g.shape[-1]).sum(0)
        danchor = torch.zeros((), dtype=g.dtype, device=g.device) if ctx.needs_input_grad[3] else None
        return dx, None, dbias, danchor, None


class _SeamLinear(torch.autograd.Function):
    """Per-example linear whose vmap rule merges the batch and taps the seam."""

    generate_vmap_rule = False

    @staticmethod
    def forward(x, W, bias):
        return F.linear(x, W) if bias is None else F.linear(x, W) + bias

    @staticmethod
    def setup_context(ctx, inputs, output):
        pass

    @staticmethod
    def backward(ctx, g):
        raise RuntimeError("the capture seam is differentiated through its vmap rule only")

    @staticmethod
    def vmap(info, in_dims, x, W, bias):
        sess = active_session()
        xd, wd, bias_d = in_dims
        if xd is None:
            x = x.unsqueeze(0).expand(info.batch_size, *x.shape)
        elif xd != 0:
            x = x.movedim(xd, 0)
        if bias is not None and bias_d is not None:
            bias = bias.movedim(bias_d, 0)
            bias = bias.view(bias.shape[0], *([1] * (x.dim() - 2)), bias.shape[-1])
        if wd is not None or sess is None or sess.mode != "capture" or id(W) not in sess.eligible:
            if wd is not None:
                out = torch.einsum("b...i,boi->b...o", x, W.movedim(wd, 0))
            else:
                out = F.linear(x, W)
            return (out if bias is None else out + bias), 0
        rec = SiteRecord(x=x, A=None, B=None, scaling=1.0, a_obj=None, b_obj=None,
                         a_transposed=False, b_transposed=False, w_obj=W)
        sess.sites.append(rec)
        return _TapLinear.apply(x, W, bias, sess.anchor, rec), 0


# ---------------------------------------------------------------------------
# Mixture-of-experts expert FFN (full expert weights)
# ---------------------------------------------------------------------------


def _dense_routing(top_k_index: torch.Tensor, top_k_weights: torch.Tensor, n_experts: int) -> torch.Tensor:
    """Per-expert routing weights [..., E]: a token's weight for each expert, 0 where not routed."""
    if top_k_weights.shape[-1] == n_experts and top_k_index.shape != top_k_weights.shape:
        return top_k_weights  # already dense
    hit = top_k_index.unsqueeze(-1) == torch.arange(n_experts, device=top_k_index.device)
    return (hit.to(top_k_weights.dtype) * top_k_weights.unsqueeze(-1)).sum(-2)


def _expert_ffn(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, batched: bool) -> torch.Tensor:
    """down(silu(gate(x)) * up(x)) for one expert; with ``batched`` the weights carry the batch axis."""
    inter = w1.shape[-2] // 2
    gu = torch.einsum("b...h,bjh->b...j", x, w1) if batched else F.linear(x, w1)
    h = F.silu(gu[..., :inter].float()).to(x.dtype) * gu[..., inter:]
    return torch.einsum("b...i,bhi->b...h", h, w2) if batched else F.linear(h, w2)


def _moe_dense(x, gate_up_proj, down_proj, top_k_index, top_k_weights, batched: bool = False):
    """Every token through every expert, weighted by its routing weight; fp32 sum over experts."""
    n_exp = gate_up_proj.shape[-3]
    w_te = _dense_routing(top_k_index, top_k_weights, n_exp)
    out = torch.zeros(x.shape, dtype=torch.float32, device=x.device)
    for e in range(n_exp):
        w1 = gate_up_proj[:, e] if batched else gate_up_proj[e]
        w2 = down_proj[:, e] if batched else down_proj[e]
        out = out + (_expert_ffn(x, w1, w2, batched) * w_te[..., e : e + 1]).float()
    return out.to(x.dtype)


def _moe_tapped(sess: CaptureSession, x, gate_up_proj, down_proj, top_k_index, top_k_weights):
    """Batch-merged MoE over the routed rows only, recording each expert's two linears.

    Rows are grouped by expert (stable, so each expert's rows stay in example
    order); every expert's rows form one segment per example, the
    per-(example, expert) groups of the reference's grouped backward
    (PAT/kernels/_grouped_moe.py:255).
    """
    from opaque_amd.engine import Segments  # the engine imports this module

    n_ex, hid = x.shape[0], x.shape[-1]
    xf = x.reshape(-1, hid)
    per = xf.shape[0] // n_ex
    k = top_k_index.shape[-1]
    idf = top_k_index.reshape(-1, k).long()
    wf = top_k_weights.reshape(-1, k)
    n_exp, two_i = gate_up_proj.shape[0], gate_up_proj.shape[1]
    inter, dt = two_i // 2, x.dtype
    hit = idf.unsqueeze(-1) == torch.arange(n_exp, device=x.device)  # [N, K, E]
    routed = hit.any(1)  # [N, E]
    counts = routed.view(n_ex, per, n_exp).sum(1).t().tolist()  # [E][n_ex], one host sync
    w_te = (hit.to(wf.dtype) * wf.unsqueeze(-1)).sum(1)  # [N, E], differentiable in the weights
    # Flat (expert, row) positions of the routed pairs, grouped by expert and
    # ascending in row within each expert.
    order = torch.argsort(routed.t().reshape(-1).logical_not().to(torch.int8), stable=True)
    out = torch.zeros(xf.shape, dtype=torch.float32, device=x.device)
    pos = 0
    n_rows_all = xf.shape[0]
    for e in range(n_exp):
        lens = counts[e]
        n_e = sum(lens)
        starts = [sum(lens[:j]) for j in range(n_ex)]
        segs = Segments(starts, list(lens), list(range(n_ex)), n_ex, max(n_e, 1))
        r1 = SiteRecord(x=None, A=None, B=None, scaling=1.0, a_obj=None, b_obj=None, a_transposed=False,
                        b_transposed=False, w_obj=gate_up_proj, w_index=e, segments=segs)
        r2 = SiteRecord(x=None, A=None, B=None, scaling=1.0, a_obj=None, b_obj=None, a_transposed=False,
                        b_transposed=False, w_obj=down_proj, w_index=e, segments=segs)
        sess.sites += [r1, r2]
        if n_e == 0:
            # One zero row stands in for the empty group: it adds nothing.
            r1.x, r1.g = xf.new_zeros(1, hid), xf.new_zeros(1, two_i)
            r2.x, r2.g = xf.new_zeros(1, inter), xf.new_zeros(1, hid)
            continue
        rows = order[pos : pos + n_e] - e * n_rows_all
        pos += n_e
        xe = xf.index_select(0, rows)
        r1.x = xe.detach()
        gu = _TapLinear.apply(xe, gate_up_proj[e], None, sess.anchor, r1)
        h = F.silu(gu[:, :inter].float()).to(dt) * gu[:, inter:]
        r2.x = h.detach()
        y = _TapLinear.apply(h, down_proj[e], None, sess.anchor, r2)
        we = w_te[:, e].index_select(0, rows)
        out = out.index_add(0, rows, (y * we.unsqueeze(-1).to(dt)).float())
    return out.to(dt).reshape(x.shape)


class _SeamMoE(torch.autograd.Function):
    """Per-example MoE expert FFN whose vmap rule merges the batch and taps every expert."""

    generate_vmap_rule = False

    @staticmethod
    def forward(x, gate_up_proj, down_proj, top_k_index, top_k_weights):
        return _moe_dense(x, gate_up_proj, down_proj, top_k_index, top_k_weights)

    @staticmethod
    def setup_context(ctx, inputs, output):
        pass

    @staticmethod
    def backward(ctx, g):
        raise RuntimeError("the capture seam is differentiated through its vmap rule only")

    @staticmethod
    def vmap(info, in_dims, x, gate_up_proj, down_proj, top_k_index, top_k_weights):
        sess = active_session()
        xd, w1d, w2d, id_d, wd = in_dims

        def front(t, d):
            return t.unsqueeze(0).expand(info.batch_size, *t.shape) if d is None else t.movedim(d, 0)

        x, top_k_index, top_k_weights = front(x, xd), front(top_k_index, id_d), front(top_k_weights, wd)
        if w1d is not None or w2d is not None:
            # Per-example (expanded) expert weights: plain batched math.
            w1, w2 = front(gate_up_proj, w1d), front(down_proj, w2d)
            return _moe_dense(x, w1, w2, top_k_index, top_k_weights, batched=True), 0
        if (sess is None or sess.mode != "capture" or id(gate_up_proj) not in sess.eligible
                or id(down_proj) not in sess.eligible):
            return _moe_dense(x, gate_up_proj, down_proj, top_k_index, top_k_weights), 0
        return _moe_tapped(sess, x, gate_up_proj, down_proj, top_k_index, top_k_weights), 0


def moe(x: torch.Tensor, gate_up_proj: torch.Tensor, down_proj: torch.Tensor,
        top_k_index: torch.Tensor, top_k_weights: torch.Tensor) -> torch.Tensor:
    """Mixture-of-experts expert FFN with stacked expert weights, clipped per (example, expert).

    Same signature and layout as the reference's ``opaque_moe``
    (PAT/kernels/moe.py:179-221; Hugging Face stacked experts):
    ``x`` [..., H], ``gate_up_proj`` [E, 2I, H] (gate rows first),
    ``down_proj`` [E, H, I], ``top_k_index`` / ``top_k_weights`` [..., K]
    (or dense [..., E] weights); out = sum_k w_k down_e(silu(gate_e(x)) *
    up_e(x)) over the routed experts e = top_k_index[k].  Outside
    ``clipped_grad`` this is plain differentiable math.  Inside it the
    expert weights' per-example gradients are never materialised: each
    expert's two linears are full-weight sites over that expert's rows, one
    segment per example, so an example's norm sums its share of every
    expert it was routed to.
    """
    sess = active_session()
    if sess is None:
        return _moe_dense(x, gate_up_proj, down_proj, top_k_index, top_k_weights)
    if sess.mode == "discover":
        for t in (gate_up_proj, down_proj):
            sess.uses[id(t)] = sess.uses.get(id(t), 0) + 1
            sess.linear_ws.append(id(t))
        return _moe_dense(x, gate_up_proj.detach(), down_proj.detach(), top_k_index, top_k_weights)
    if id(gate_up_proj) not in sess.eligible and id(down_proj) not in sess.eligible:
        return _moe_dense(x, gate_up_proj, down_proj, top_k_index, top_k_weights)
    return _SeamMoE.apply(x, gate_up_proj, down_proj, top_k_index, top_k_weights)


def linear(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``x W^T + bias`` whose weight gradient the DP engine clips without materialising it.

    Outside ``clipped_grad`` this is ``torch.nn.functional.linear``.
    """
    sess = active_session()
    if sess is None:
        return F.linear(x, W, bias)
    if sess.mode == "discover":
        sess.uses[id(W)] = sess.uses.get(id(W), 0) + 1
        sess.linear_ws.append(id(W))
        return F.linear(x, W.detach(), bias)
    if id(W) not in sess.eligible:
        return F.linear(x, W, bias)
    return _SeamLinear.apply(x, W, bias)


class Linear(torch.nn.Linear):
    """``torch.nn.Linear`` routed through the full-weight seam."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return linear(x, self.weight, self.bias)


def lora_linear(x: torch.Tensor, W: torch.Tensor, A: torch.Tensor, B: torch.Tensor,
                scaling: float, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``x W^T + bias + scaling (x A) B`` with A [d_in, r], B [r, d_out].

    Same computation as the reference's ``Opaque_LoRA_W`` (lora.py:217-293).
    """
    return _lora(x, W, A, B, scaling, bias, A, B, False, False)


def peft_lora_linear(x: torch.Tensor, W: torch.Tensor, lora_A_weight: torch.Tensor,
                     lora_B_weight: torch.Tensor, scaling: float,
                     bias: torch.Tensor | None = None) -> torch.Tensor:
    """LoRA with PEFT's storage: lora_A.weight [r, d_in], lora_B.weight [d_out, r].

    The reference transposes these before its kernels (PAT/peft/components/linear.py:60-65).
    """
    return _lora(x, W, lora_A_weight.t(), lora_B_weight.t(), scaling, bias,
                 lora_A_weight, lora_B_weight, True, True)


class LoRALinear(torch.nn.Module):
    """A frozen ``Linear`` with a trainable LoRA adapter routed through the seam.

    Parameters ``lora_A`` [r, in] and ``lora_B`` [out, r] use PEFT's layout;
    ``scaling = alpha / r`` as in PEFT (PAT/peft/components/_utils.py:43).
    """

    def __init__(self, in_features: int, out_features: int, r: int, alpha: float = 16.0,
                 bias: bool = False, device=None, dtype=None) -> None:
        super().__init__()
        kw = {"device": device, "dtype": dtype}
        self.weight = torch.nn.Parameter(torch.empty(out_features, in_features, **kw), requires_grad=False)
        self.bias = torch.nn.Parameter(torch.zeros(out_features, **kw), requires_grad=False) if bias else None
        self.lora_A = torch.nn.Parameter(torch.empty(r, in_features, **kw))
        self.lora_B = torch.nn.Parameter(torch.zeros(out_features, r, **kw))
        self.scaling = alpha / r
        torch.nn.init.kaiming_uniform_(self.weight, a=5**0.5)
        torch.nn.init.kaiming_uniform_(self.lora_A, a=5**0.5)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return peft_lora_linear(x, self.weight, self.lora_A, self.lora_B, self.scaling, self.bias)

    @classmethod
    def from_linear(cls, base: torch.nn.Linear, r: int, alpha: float = 16.0) -> LoRALinear:
        """Wrap an existing ``Linear``: its weight and bias become the frozen base (shared, not copied)."""
        m = cls.__new__(cls)
        torch.nn.Module.__init__(m)
        w = base.weight
        m.weight = torch.nn.Parameter(w.data, requires_grad=False)
        m.bias = None if base.bias is None else torch.nn.Parameter(base.bias.data, requires_grad=False)
        m.lora_A = torch.nn.Parameter(torch.empty(r, base.in_features, device=w.device, dtype=w.dtype))
        m.lora_B = torch.nn.Parameter(torch.zeros(base.out_features, r, device=w.device, dtype=w.dtype))
        m.scaling = alpha / r
        torch.nn.init.kaiming_uniform_(m.lora_A, a=5**0.5)
        return m


def _replace_linears(model: torch.nn.Module, targets, make) -> list[str]:
    names = []
    for name, mod in list(model.named_modules()):
        for child_name, child in list(mod.named_children()):
            if type(child) is torch.nn.Linear and child_name in targets:
                setattr(mod, child_name, make(child))
                names.append(f"{name}.{child_name}" if name else child_name)
    return names


def inject_lora(model: torch.nn.Module, target_modules=("q_proj", "k_proj", "v_proj", "o_proj",
                                                        "gate_proj", "up_proj", "down_proj"),
                r: int = 8, alpha: float = 16.0, freeze_base: bool = True) -> list[str]:
    """Give every ``nn.Linear`` child named in ``target_modules`` a LoRA adapter routed through the seam.

    The counterpart of building a PEFT LoRA model and installing the
    reference's patched forward (``apply_peft_model_patches``,
    PAT/peft/_router.py:158-198, which routes ``lora_A``/``lora_B`` into
    ``Opaque_LoRA_W``): each matching ``Linear`` becomes a ``LoRALinear``
    sharing its weight and bias, ``lora_A`` Kaiming-initialised and
    ``lora_B`` zero as in PEFT.  With ``freeze_base`` every parameter of the
    model other than the adapters stops requiring grad.  Returns the
    replaced modules' names.
    """
    if freeze_base:
        for p in model.parameters():
            p.requires_grad_(False)
    return _replace_linears(model, set(target_modules), lambda lin: LoRALinear.from_linear(lin, r, alpha))


def route_linears(model: torch.nn.Module, target_modules) -> list[str]:
    """Route the named ``nn.Linear`` children through the full-weight seam (parameters shared)."""
    def make(lin: torch.nn.Linear) -> Linear:
        m = Linear.__new__(Linear)
        torch.nn.Module.__init__(m)
        m.in_features, m.out_features = lin.in_features, lin.out_features
        m.weight, m.bias = lin.weight, lin.bias
        return m

    return _replace_linears(model, set(target_modules), make)


__all__ = [
    "CaptureSession",
    "Linear",
    "LoRALinear",
    "SiteRecord",
    "active_session",
    "inject_lora",
    "linear",
    "lora_linear",
    "moe",
    "peft_lora_linear",
    "route_linears",
]
