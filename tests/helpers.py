"""Shared fixtures for the parity tests: seeded synthetic inputs and metrics."""
from __future__ import annotations

import numpy as np

from air_amd import capi, quant

BLOCK = {capi.TYPE_Q8_0: (32, 34), capi.TYPE_Q4_0: (32, 18), capi.TYPE_Q4_K: (256, 144)}


def weights(type_id: int, k: int, n: int, seed: int) -> np.ndarray:
    return quant.synthetic_weights(type_id, k, n, seed)


def activations(m: int, k: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((m, k), dtype=np.float32)


def random_blocks(type_id: int, blocks: int, seed: int, finite_scales: bool = True) -> np.ndarray:
    """Random canonical blocks: random code bytes, and random f16 scales
    (finite, normal or subnormal, either sign) unless finite_scales=False."""
    rng = np.random.default_rng(seed)
    _, bb = BLOCK[type_id]
    raw = rng.integers(0, 256, size=(blocks, bb), dtype=np.uint8)
    nscales = 2 if type_id == capi.TYPE_Q4_K else 1
    if finite_scales:
        for s in range(nscales):
            bits = rng.integers(0, 0x7C00, size=blocks, dtype=np.uint16)  # finite magnitudes
            bits |= (rng.integers(0, 2, size=blocks, dtype=np.uint16) << 15)
            raw[:, 2 * s:2 * s + 2] = bits.view(np.uint8).reshape(blocks, 2)
    return raw.reshape(-1)


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    denom = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / (denom if denom > 0 else 1.0))


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit equality for non-NaN values; NaN positions must agree."""
    a = np.asarray(a, dtype=np.float32).reshape(-1)
    b = np.asarray(b, dtype=np.float32).reshape(-1)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return bool(np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))
