"""Keep bits of the fused kernels' attention dropout, restated on the CPU.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference drops attention probabilities with ``nn.Dropout``
(src/deberta/modeling/deberta_v2_native.py:222, 636): ``probs * keep / (1 -
p)`` with ``keep`` drawn from torch's generator, which a fused kernel cannot
reproduce.  The kernels draw ``keep`` from Philox4x32-10 (J. K. Salmon, M. A.
Moraes, R. O. Dror, D. E. Shaw, "Parallel random numbers: as easy as 1, 2,
3", SC 2011) keyed by a per-call 64-bit seed; this module restates that
contract (deberta_amd/csrc/dsa_dropout.h) in numpy, so that the parity tests
can hand the same mask to ``oracle.eager.attend`` (which applies it as the
reference's dropout does).  For pair (i, j) of head h, batch row b, with
r = j % 64, jb = r // 16, g = (r % 16) // 4, e = r % 4:

    counter = ((j // 64) * 8 + g * 2 + jb // 2, i, h, b)
    key     = (seed & 0xffffffff, seed >> 32)
    x       = Philox4x32-10(counter, key)
    u       = (jb % 2) * 4 + e;   v = (x[u // 2] >> (16 * (u % 2))) & 0xffff
    keep    = v >= t            (t = round(p * 65536), in [1, 65535])

The Philox function is pinned by the published known-answer vectors of
Philox4x32-10 (tests/test_oracle_dropout.py).
"""

from __future__ import annotations

import numpy as np

_M0, _M1 = 0xD2511F53, 0xCD9E8D57  # round multipliers
_W0, _W1 = 0x9E3779B9, 0xBB67AE85  # key-schedule increments
_MASK32 = 0xFFFFFFFF


def philox4x32_10(counter: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x32 with ten rounds on ``counter`` (``(..., 4)`` unsigned
    32-bit words) under ``key`` (two 32-bit words); returns ``(..., 4)``
    uint32.  Round: ``(hi0, lo0) = M0 * c0``, ``(hi1, lo1) = M1 * c2``,
    ``c <- (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0)``, then the key gains
    the Weyl increments."""
    c = np.asarray(counter, dtype=np.uint64) & np.uint64(_MASK32)
    c0, c1, c2, c3 = (c[..., n] for n in range(4))
    k0, k1 = int(key[0]) & _MASK32, int(key[1]) & _MASK32
    m32 = np.uint64(_MASK32)
    for _ in range(10):
        p0 = np.uint64(_M0) * c0  # 32 x 32 bits: exact in 64
        p1 = np.uint64(_M1) * c2
        hi0, lo0 = p0 >> np.uint64(32), p0 & m32
        hi1, lo1 = p1 >> np.uint64(32), p1 & m32
        c0, c1, c2, c3 = hi1 ^ c1 ^ np.uint64(k0), lo1, hi0 ^ c3 ^ np.uint64(k1), lo0
        k0 = (k0 + _W0) & _MASK32
        k1 = (k1 + _W1) & _MASK32
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def keep_mask(seed: int, threshold: int, B: int, H: int, Lq: int, Lk: int) -> np.ndarray:
    """The kernels' keep mask, bool ``[B, H, Lq, Lk]`` (True = kept), for a
    call with this seed and threshold."""
    if not 1 <= threshold <= 65535:
        raise ValueError(f"threshold must be in [1, 65535], got {threshold}")
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    nkt = (Lk + 63) // 64
    b, h, i, kt, g, half = np.meshgrid(
        np.arange(B), np.arange(H), np.arange(Lq), np.arange(nkt), np.arange(4), np.arange(2), indexing="ij"
    )
    ctr = np.stack([kt * 8 + g * 2 + half, i, h, b], axis=-1)
    x = philox4x32_10(ctr, (seed & _MASK32, seed >> 32))  # (B, H, Lq, nkt, 4 g, 2 half, 4 words)
    lo, hi = x & np.uint32(0xFFFF), x >> np.uint32(16)
    vals = np.stack([lo, hi], axis=-1).reshape(B, H, Lq, nkt, 4, 2, 2, 4)  # (..., g, half, kb, e): u = 4 kb + e
    keep = vals >= threshold
    # key j % 64 = 16 (2 half + kb) + 4 g + e
    keep = keep.transpose(0, 1, 2, 3, 5, 6, 4, 7).reshape(B, H, Lq, nkt * 64)
    return keep[..., :Lk]
