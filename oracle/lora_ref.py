"""fp64 per-example gradients of LoRA and full-weight linears (test oracle).

Restates the per-sample formulas of opaque-patches/.../kernels/lora.py:164-176
(dA[i] = s X[i]^T (G[i] B^T), dB[i] = s (X[i] A)^T G[i]) with explicit
segments, and the per-example full-weight gradient G[i]^T X[i] whose squared
Frobenius norm the Gram form computes as sum_{t,s}(g_t.g_s)(x_t.x_s).
"""

from __future__ import annotations

import torch


def lora_per_example(X, G, A, B, scaling, starts, lengths):
    """Returns (dA [n_seg, d_in, r], dB [n_seg, r, d_out]) in float64."""
    X64, G64, A64, B64 = (t.double() for t in (X, G, A, B))
    dA, dB = [], []
    for s, ln in zip(starts, lengths):
        x, g = X64[s : s + ln], G64[s : s + ln]
        dA.append(scaling * x.T @ (g @ B64.T))
        dB.append(scaling * (x @ A64).T @ g)
    return torch.stack(dA), torch.stack(dB)


def linear_per_example(X, G, starts, lengths):
    """Per-example full-weight gradients G[i]^T X[i], [n_seg, d_out, d_in] float64."""
    X64, G64 = X.double(), G.double()
    return torch.stack([G64[s : s + ln].T @ X64[s : s + ln] for s, ln in zip(starts, lengths)])


def linear_sqnorm_gram(X, G, starts, lengths):
    """sum_{t,s} (g_t . g_s)(x_t . x_s) per segment, float64."""
    X64, G64 = X.double(), G.double()
    out = []
    for s, ln in zip(starts, lengths):
        x, g = X64[s : s + ln], G64[s : s + ln]
        out.append(((x @ x.T) * (g @ g.T)).sum())
    return torch.stack(out)
