"""Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11), vectorised in numpy.

The same counter-based generator the kernels use: counter (c0, step_lo,
step_hi, purpose), key (seed_lo, seed_hi), uniform = (word >> 8) * 2^-24.
Host callers use it to derive per-request uniforms that do not depend on a
request's position in the batch.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np

_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key: np.ndarray) -> np.ndarray:
    """ctr [..., 4] uint32, key [..., 2] uint32 → [..., 4] uint32."""
    c = [ctr[..., i].astype(np.uint32) for i in range(4)]
    k0 = key[..., 0].astype(np.uint32).copy()
    k1 = key[..., 1].astype(np.uint32).copy()
    with np.errstate(over="ignore"):
        for r in range(10):
            if r > 0:
                k0 = k0 + _W0
                k1 = k1 + _W1
            p0 = _M0 * c[0].astype(np.uint64)
            p1 = _M1 * c[2].astype(np.uint64)
            hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
            lo0 = (p0 & _MASK).astype(np.uint32)
            hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
            lo1 = (p1 & _MASK).astype(np.uint32)
            c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return np.stack(c, axis=-1)


def philox_uniforms(seeds: Sequence[int], rows: Sequence[int], steps: Sequence[int],
                    purpose: int = 0, word: int = 0) -> np.ndarray:
    seeds = np.asarray([int(s) & 0xFFFFFFFFFFFFFFFF for s in seeds], dtype=np.uint64)
    rows = np.asarray([int(r) & 0xFFFFFFFF for r in rows], dtype=np.uint64)
    steps = np.asarray([int(s) & 0xFFFFFFFFFFFFFFFF for s in steps], dtype=np.uint64)
    n = seeds.size
    ctr = np.zeros((n, 4), dtype=np.uint32)
    ctr[:, 0] = rows.astype(np.uint32)
    ctr[:, 1] = (steps & _MASK).astype(np.uint32)
    ctr[:, 2] = (steps >> np.uint64(32)).astype(np.uint32)
    ctr[:, 3] = purpose
    key = np.zeros((n, 2), dtype=np.uint32)
    key[:, 0] = (seeds & _MASK).astype(np.uint32)
    key[:, 1] = (seeds >> np.uint64(32)).astype(np.uint32)
    w = philox4x32_10(ctr, key)[:, word]
    return ((w >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)
