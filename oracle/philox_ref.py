"""Philox4x32-10 and the device noise transform, in numpy (test oracle).

Philox4x32-10 follows Salmon, Moraes, Dror and Shaw, "Parallel random
numbers: as easy as 1, 2, 3" (SC 2011): 10 rounds of
  (c0,c1,c2,c3) <- (hi(M1*c2)^c1^k0, lo(M1*c2), hi(M0*c0)^c3^k1, lo(M0*c0))
with the key bumped by the Weyl constants between rounds.  The transform
restates the inverse-CDF sampler of opaque-dpsgd/.../noise/_gaussian.py:
252-266 in float64 (the device evaluates it in float32).
"""

from __future__ import annotations

import numpy as np
from scipy.special import erfinv

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint64(0x9E3779B9), np.uint64(0xBB67AE85)
MASK = np.uint64(0xFFFFFFFF)

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


def words_for_elements(seed: int, flat_offset: int, n: int, tag: int = 0) -> np.ndarray:
    """uint32 word used by each element e = flat_offset + i: word (e & 3) of block e >> 2."""
    e = np.arange(flat_offset, flat_offset + n, dtype=np.uint64)
    q = e >> np.uint64(2)
    w = philox4x32_10(q & MASK, q >> np.uint64(32), np.uint64(tag), np.uint64(0),
                      np.uint64(seed & 0xFFFFFFFF), np.uint64(seed >> 32))
    stacked = np.stack(w, axis=-1)
    return stacked[np.arange(n), (e & np.uint64(3)).astype(np.int64)]


def uniforms(words: np.ndarray) -> np.ndarray:
    """float32 uniforms (x >> 8) * 2^-24 clamped to [eps, 1 - eps], as float64."""
    u = (words >> np.uint32(8)).astype(np.float64) * 2.0**-24
    eps = float(np.finfo(np.float32).eps)
    return np.clip(u, eps, 1.0 - eps)


def gaussian_noise(center: np.ndarray, sigma: float, seed: int, flat_offset: int = 0, tag: int = 0) -> np.ndarray:
    """center + sigma*sqrt(2)*erfinv(2u - 1) in float64 for the device stream."""
    c = np.asarray(center, dtype=np.float64).reshape(-1)
    if sigma == 0.0:
        return c.copy()
    u = uniforms(words_for_elements(seed, flat_offset, c.size, tag))
    return c + sigma * np.sqrt(2.0) * erfinv(2.0 * u - 1.0)
