"""Immutable RNG keys with the reference's derivation rules.

``key``/``fold_in``/``split`` reproduce ``opaque-engine/.../random/_engine.py:
27-101`` bit for bit: a key is a 64-bit seed; folding mixes the seed and each
datum with an 8-byte BLAKE2b digest (ints as 16-byte little-endian signed,
strings as UTF-8, each part followed by ``b"|"``).  The per-step noise key of
the DP step is ``fold_in(key, step)`` as in the reference; its 64-bit seed
keys the device Philox stream.
"""

from __future__ import annotations

import dataclasses
import hashlib

import torch

_U64 = (1 << 64) - 1
_MAX_TORCH_SEED = 2**63 - 1


def _digest64(*parts: object) -> int:
    h = hashlib.blake2b(digest_size=8)
    for part in parts:
        if isinstance(part, int):
            h.update(int(part).to_bytes(16, byteorder="little", signed=True))
        else:
            h.update(str(part).encode("utf-8"))
        h.update(b"|")
    return int.from_bytes(h.digest(), byteorder="little", signed=False)


@dataclasses.dataclass(frozen=True)
class RngKey:
    """Immutable RNG key: a 64-bit ``seed`` and an implementation tag."""

    seed: int
    impl: str = "opaque_threefry_like"


def key(seed: int) -> RngKey:
    if not isinstance(seed, int):
        raise TypeError(f"seed must be int, got {type(seed)}")
    return RngKey(seed=seed & _U64)


def fold_in(rng_key: RngKey, *data: int | str) -> RngKey:
    if not data:
        raise ValueError("fold_in requires at least one data argument")
    out = rng_key
    for d in data:
        if not isinstance(d, (int, str)):
            raise TypeError(f"data must be int or str, got {type(d)}")
        out = RngKey(seed=_digest64(out.seed, d), impl=out.impl)
    return out


def split(rng_key: RngKey, num: int = 2) -> tuple[RngKey, ...]:
    if num < 1:
        raise ValueError(f"num must be >= 1, got {num}")
    return tuple(fold_in(rng_key, i) for i in range(num))


def generator_from_key(rng_key: RngKey) -> torch.Generator:
    """Seeded CPU ``torch.Generator`` (for callers that need one)."""
    return torch.Generator().manual_seed(rng_key.seed % _MAX_TORCH_SEED)


def random_key() -> RngKey:
    """A key seeded from the OS entropy pool (not reproducible)."""
    import secrets

    return key(secrets.randbits(64))


__all__ = ["RngKey", "fold_in", "generator_from_key", "key", "random_key", "split"]
