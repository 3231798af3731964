"""Host-side JAX-compatible key plumbing (threefry2x32, partitionable mode).

Keys are uint32 pairs, the data of a `jax.random.key` under the default
threefry2x32 implementation with jax_threefry_partitionable=True (the mode the
reference's kernels require, src/nanorts/core/reservations.py:309-315):
  key(seed)          = (seed >> 32, seed & 0xFFFFFFFF)
  fold_in(k, d)      = threefry(k, (0, d))
  split(k, n)[i]     = threefry(k, (0, i))
Vectorised with numpy so a batch of env roots is derived in one call.
"""
from __future__ import annotations

import numpy as np

_ROTATIONS = ((13, 15, 26, 6), (17, 29, 16, 24))
_PARITY = np.uint32(0x1BD11BDA)


def _rotl(x: np.ndarray, d: int) -> np.ndarray:
    return (x << np.uint32(d)) | (x >> np.uint32(32 - d))


def threefry2x32(key: np.ndarray, x0: np.ndarray, x1: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Threefry-2x32 with 20 rounds (Salmon et al., Random123) on broadcast arrays."""
    key = np.asarray(key, np.uint32)
    k0, k1 = key[..., 0], key[..., 1]
    ks = (k0, k1, k0 ^ k1 ^ _PARITY)
    with np.errstate(over="ignore"):
        x0 = np.asarray(x0, np.uint32) + ks[0]
        x1 = np.asarray(x1, np.uint32) + ks[1]
        for block in range(5):
            for r in _ROTATIONS[block % 2]:
                x0 = x0 + x1
                x1 = _rotl(x1, r)
                x1 = x1 ^ x0
            x0 = x0 + ks[(block + 1) % 3]
            x1 = x1 + ks[(block + 2) % 3] + np.uint32(block + 1)
    return x0, x1


def key(seed: int) -> np.ndarray:
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return np.asarray([(seed >> 32) & 0xFFFFFFFF, seed & 0xFFFFFFFF], np.uint32)


def fold_in(k: np.ndarray, data) -> np.ndarray:
    data = np.asarray(data).astype(np.int64).astype(np.uint32)
    y0, y1 = threefry2x32(np.asarray(k, np.uint32), np.zeros_like(data), data)
    return np.stack([y0, y1], axis=-1)


def split(k: np.ndarray, n: int = 2) -> np.ndarray:
    return fold_in(np.asarray(k, np.uint32), np.arange(n, dtype=np.uint32))
