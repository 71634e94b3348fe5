"""Philox4x32-10 counter-based generator and the attention-dropout keep mask.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Philox4x32-10 is the generator of J. K. Salmon, M. A. Moraes, R. O. Dror and
D. E. Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11 (the Random123
library): a 4 x 32-bit counter and a 2 x 32-bit key, ten rounds of
  (hi0, lo0) = M0 * c0,  (hi1, lo1) = M1 * c2   (32 x 32 -> 64-bit products)
  c = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0)
with the key bumped by the Weyl constants (W0, W1) between rounds.  Pinned by
the published known-answer vectors (tests/test_dropout_cpu.py).

The reference applies ``nn.Dropout`` to the softmax weights of every query's
taps (infinity/video/attention.py:80, :180).  PyTorch's own random stream
cannot be reproduced, so the HIP kernels draw the keep mask from this
generator: tap k of query row r (global token row b*N + n) and head m is
dropped when the first output word for counter (k, r mod 2^32, (r >> 32) << 16
| m, offset) under key (seed mod 2^32, seed >> 32) is below
threshold = floor(p * 2^32); kept weights are scaled by fp32 1 / (1 - p), as
``nn.Dropout`` does.
"""

from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
_MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Vectorised Philox4x32-10; arguments are uint32 arrays (broadcast)."""
    c0, c1, c2, c3 = (np.asarray(x, dtype=np.uint32) for x in (c0, c1, c2, c3))
    k0 = np.asarray(k0, dtype=np.uint32)
    k1 = np.asarray(k1, dtype=np.uint32)
    c0, c1, c2, c3, k0, k1 = np.broadcast_arrays(c0, c1, c2, c3, k0, k1)
    c0, c1, c2, c3, k0, k1 = (x.copy() for x in (c0, c1, c2, c3, k0, k1))
    with np.errstate(over="ignore"):
        for r in range(10):
            if r:
                k0 = k0 + W0
                k1 = k1 + W1
            p0 = M0 * c0.astype(np.uint64)
            p1 = M1 * c2.astype(np.uint64)
            hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
            lo0 = (p0 & _MASK32).astype(np.uint32)
            hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
            lo1 = (p1 & _MASK32).astype(np.uint32)
            c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return c0, c1, c2, c3


def dropout_threshold(p: float) -> int:
    """Drop a tap when its 32-bit draw is below this value (floor(p * 2^32))."""
    if not 0.0 <= p < 1.0:
        raise ValueError(f"dropout probability must be in [0, 1), got {p}")
    return min(int(np.floor(np.float64(p) * 4294967296.0)), 0xFFFFFFFF)


def keep_mask(p: float, seed: int, offset: int, rows, heads: int, taps: int) -> np.ndarray:
    """Boolean keep mask [len(rows), heads, taps] for global token rows ``rows``."""
    rows = np.asarray(rows, dtype=np.uint64).reshape(-1, 1, 1)
    m = np.arange(heads, dtype=np.uint64).reshape(1, -1, 1)
    k = np.arange(taps, dtype=np.uint32).reshape(1, 1, -1)
    c1 = (rows & _MASK32).astype(np.uint32)
    c2 = (((rows >> np.uint64(32)) << np.uint64(16)) | m).astype(np.uint32)
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    out = philox4x32_10(k, c1, c2, np.uint32(offset & 0xFFFFFFFF), np.uint32(seed & 0xFFFFFFFF),
                        np.uint32(seed >> 32))[0]
    return out >= np.uint32(dropout_threshold(p))


def dropout_scale(p: float) -> np.float32:
    """fp32 scale of kept weights, 1 / (1 - p) evaluated in fp32."""
    return np.float32(1.0) / (np.float32(1.0) - np.float32(p))
