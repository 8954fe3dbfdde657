"""Philox4x32-10 and the device noise transform, in numpy (test oracle).

Philox4x32-10 follows Salmon, Moraes, Dror and Shaw, "Parallel random
numbers: as easy as 1, 2, 3" (SC 2011): 10 rounds of
  (c0,c1,c2,c3) <- (hi(M1*c2)^c1^k0, lo(M1*c2), hi(M0*c0)^c3^k1, lo(M0*c0))
with the key bumped by the Weyl constants between rounds.  The transforms
restate the inverse-CDF sampler of opaque-dpsgd/.../noise/_gaussian.py:
235-278 in float64 (the device evaluates it in float32, or float64 for
compute_dtype=float64), fed by the device's uniforms:

* float32 compute: element e takes the 24-bit integer k = bits
  [24 (e mod 16), + 24) of the 384-bit string of the Philox outputs for
  counters 3 (e >> 4) + b, b = 0, 1, 2 (words in order, bit 0 first), and
  u = k 2^-24 (the grid of a float32 torch.rand);
* float64 compute: u = (w >> 11) 2^-53 with w the 64-bit word pair
  2 (e & 1) + 1 : 2 (e & 1) of block e >> 1.

A counter is {c (64-bit), tag, 0}; the key is the 64-bit seed.
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf, erfinv

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint64(0x9E3779B9), np.uint64(0xBB67AE85)
MASK = np.uint64(0xFFFFFFFF)
EPS32 = float(np.finfo(np.float32).eps)
EPS64 = float(np.finfo(np.float64).eps)

# Random123 known-answer vectors for philox4x32_10: (counter, key, output).
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    (
        (0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF),
        (0xFFFFFFFF, 0xFFFFFFFF),
        (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD),
    ),
    (
        (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
        (0xA4093822, 0x299F31D0),
        (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1),
    ),
]


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Vectorised Philox4x32-10 on uint32-valued arrays; returns 4 uint32 arrays."""
    c = [np.asarray(v, dtype=np.uint64) & MASK for v in (c0, c1, c2, c3)]
    k0 = np.asarray(k0, dtype=np.uint64) & MASK
    k1 = np.asarray(k1, dtype=np.uint64) & MASK
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        c = [
            ((p1 >> np.uint64(32)) ^ c[1] ^ k0) & MASK,
            p1 & MASK,
            ((p0 >> np.uint64(32)) ^ c[3] ^ k1) & MASK,
            p0 & MASK,
        ]
        k0 = (k0 + W0) & MASK
        k1 = (k1 + W1) & MASK
    return [v.astype(np.uint32) for v in c]


def _blocks(seed: int, ctr: np.ndarray, tag: int) -> np.ndarray:
    """[len(ctr), 4] uint32 Philox outputs for 64-bit counters ctr."""
    ctr = ctr.astype(np.uint64)
    w = philox4x32_10(ctr & MASK, ctr >> np.uint64(32), np.uint64(tag), np.uint64(0),
                      np.uint64(seed & 0xFFFFFFFF), np.uint64(seed >> 32))
    return np.stack(w, axis=-1)


def uniform24_for_elements(seed: int, flat_offset: int, n: int, tag: int = 0) -> np.ndarray:
    """The 24-bit integer k of each element e = flat_offset + i (float32 compute)."""
    e = np.arange(flat_offset, flat_offset + n, dtype=np.int64)
    g = e >> 4
    groups = np.unique(g)
    words = _blocks(seed, (3 * groups[:, None] + np.arange(3)[None, :]).reshape(-1), tag)
    words = words.reshape(len(groups), 12).astype(np.uint64)  # 12 words = 384 bits per group
    row = np.searchsorted(groups, g)
    bit = 24 * (e & 15)
    wi, sh = bit >> 5, (bit & 31).astype(np.uint64)
    lo = words[row, wi] >> sh
    nxt = np.minimum(wi + 1, 11)
    hi = np.where(sh > 8, words[row, nxt] << (np.uint64(32) - sh), np.uint64(0))
    return ((lo | hi) & np.uint64(0xFFFFFF)).astype(np.int64)


def uniform53_for_elements(seed: int, flat_offset: int, n: int, tag: int = 0) -> np.ndarray:
    """The 53-bit integer k of each element (float64 compute), as float64-exact ints."""
    e = np.arange(flat_offset, flat_offset + n, dtype=np.int64)
    w = _blocks(seed, e >> 1, tag).astype(np.uint64)
    h = (e & 1) * 2
    lo, hi = w[np.arange(n), h], w[np.arange(n), h + 1]
    return ((hi << np.uint64(32)) | lo) >> np.uint64(11)


def uniforms(k: np.ndarray, bits: int = 24) -> np.ndarray:
    """u = k 2^-bits clamped to [eps, 1 - eps] of the compute dtype (float64 values)."""
    eps = EPS32 if bits == 24 else EPS64
    u = np.asarray(k, dtype=np.float64) * 2.0**-bits
    return np.clip(u, eps, 1.0 - eps)


def gaussian_noise(center: np.ndarray, sigma: float, seed: int, flat_offset: int = 0, tag: int = 0,
                   wide: bool = False) -> np.ndarray:
    """center + sigma*sqrt(2)*erfinv(2u - 1) in float64 for the device stream
    (_gaussian.py:262-266)."""
    c = np.asarray(center, dtype=np.float64).reshape(-1)
    if sigma == 0.0:
        return c.copy()
    if wide:
        u = uniforms(uniform53_for_elements(seed, flat_offset, c.size, tag), 53)
    else:
        u = uniforms(uniform24_for_elements(seed, flat_offset, c.size, tag), 24)
    return c + sigma * np.sqrt(2.0) * erfinv(2.0 * u - 1.0)


def gaussian_noise_bounded(center: np.ndarray, sigma: float, low: float, high: float, seed: int,
                           flat_offset: int = 0, tag: int = 0, wide: bool = False) -> np.ndarray:
    """The bounded Gaussian of _gaussian.py:267-276 in float64: the uniform
    renormalised to [Phi(z_low), Phi(z_high)], clamped to [eps, 1 - eps],
    mapped through the inverse CDF and clamped to [low, high]; sigma == 0
    clamps the centre (_gaussian.py:245-250)."""
    c = np.asarray(center, dtype=np.float64).reshape(-1)
    if sigma == 0.0:
        return np.clip(c, low, high)
    if wide:
        raw, eps = uniform53_for_elements(seed, flat_offset, c.size, tag) * 2.0**-53, EPS64
    else:
        raw, eps = uniform24_for_elements(seed, flat_offset, c.size, tag) * 2.0**-24, EPS32
    z_low, z_high = (low - c) / sigma, (high - c) / sigma
    alpha = 0.5 * (1.0 + erf(z_low / np.sqrt(2.0)))
    beta = 0.5 * (1.0 + erf(z_high / np.sqrt(2.0)))
    u = np.clip(alpha + raw * (beta - alpha), eps, 1.0 - eps)
    return np.clip(c + sigma * np.sqrt(2.0) * erfinv(2.0 * u - 1.0), low, high)
