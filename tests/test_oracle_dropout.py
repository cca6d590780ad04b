"""The CPU restatement of the kernels' dropout keep bits (oracle/dropout.py)
and the oracle's dropout step, pinned without the GPU.

* Philox4x32-10 against the published known-answer vectors of the
  generator (Random123's test vectors for philox4x32 with 10 rounds).
* The vectorised mask against a scalar evaluation of the stated contract,
  element by element, on a ragged shape.
* The kept fraction against 1 - t / 65536 (binomial bound), and different
  seeds, heads and batch rows giving different masks.
* ``oracle.eager.attend`` with a mask given equals the reference's
  ``nn.Dropout`` step (deberta_v2_native.py:636) with torch's own mask.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import eager
from oracle.dropout import keep_mask, philox4x32_10

KAT = [  # (counter, key, output), philox4x32 with 10 rounds
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    (
        (0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344),
        (0xA4093822, 0x299F31D0),
        (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1),
    ),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = philox4x32_10(np.array(ctr, dtype=np.uint64), key)
    assert tuple(int(x) for x in got) == want


def test_philox_batched_equals_single():
    rng = np.random.default_rng(0)
    ctr = rng.integers(0, 1 << 32, size=(5, 3, 4), dtype=np.uint64)
    got = philox4x32_10(ctr, (0xDEADBEEF, 0x01234567))
    for idx in np.ndindex(5, 3):
        assert np.array_equal(got[idx], philox4x32_10(ctr[idx], (0xDEADBEEF, 0x01234567)))


def _scalar_keep(seed: int, t: int, b: int, h: int, i: int, j: int) -> bool:
    """The contract of deberta_amd/csrc/dsa_dropout.h for one pair."""
    r = j % 64
    jb, g, e = r // 16, (r % 16) // 4, r % 4
    ctr = np.array([(j // 64) * 8 + g * 2 + jb // 2, i, h, b], dtype=np.uint64)
    x = philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))
    u = (jb % 2) * 4 + e
    v = (int(x[u // 2]) >> (16 * (u % 2))) & 0xFFFF
    return v >= t


def test_mask_equals_scalar_contract():
    seed, t = 0x0123_4567_89AB_CDEF, 6554
    B, H, Lq, Lk = 2, 3, 37, 150
    m = keep_mask(seed, t, B, H, Lq, Lk)
    assert m.shape == (B, H, Lq, Lk) and m.dtype == bool
    rng = np.random.default_rng(1)
    picks = [(b, h, i, j) for b in range(B) for h in range(H) for i in (0, 17, Lq - 1) for j in range(0, Lk, 1)]
    picks = [picks[n] for n in rng.choice(len(picks), 400, replace=False)]
    for b, h, i, j in picks:
        assert m[b, h, i, j] == _scalar_keep(seed, t, b, h, i, j), (b, h, i, j)


@pytest.mark.parametrize("t", [1, 6554, 32768, 65535])
def test_kept_fraction(t):
    m = keep_mask(0xA5A5_0001, t, 2, 4, 128, 256)
    n = m.size
    q = t / 65536
    sigma = math.sqrt(q * (1 - q) / n)
    assert abs((1 - m.mean()) - q) <= 6 * sigma + 1.0 / n


def test_masks_differ_across_seeds_heads_and_rows():
    a = keep_mask(1, 32768, 2, 2, 64, 64)
    b = keep_mask(2, 32768, 2, 2, 64, 64)
    assert (a != b).mean() > 0.4
    assert (a[0, 0] != a[0, 1]).mean() > 0.4 and (a[0, 0] != a[1, 0]).mean() > 0.4
    assert (a[0, 0, :-1] != a[0, 0, 1:]).mean() > 0.4  # neighbouring queries
    assert (a[0, 0, :, :-1] != a[0, 0, :, 1:]).mean() > 0.4  # neighbouring keys


def test_threshold_range():
    with pytest.raises(ValueError):
        keep_mask(0, 0, 1, 1, 4, 4)
    with pytest.raises(ValueError):
        keep_mask(0, 65536, 1, 1, 4, 4)


def test_attend_dropout_step_is_nn_dropout():
    """attend(dropout_keep=m, dropout_p=p) equals the reference's chain with
    nn.Dropout's own output in place of the probabilities (same mask)."""
    g = torch.Generator().manual_seed(3)
    B, H, L, D = 2, 2, 24, 16
    q, k, v = (torch.randn(B, H, L, D, generator=g, dtype=torch.float64) for _ in range(3))
    p = 0.25
    torch.manual_seed(11)
    ones = torch.nn.functional.dropout(torch.ones(B, H, L, L, dtype=torch.float64), p, training=True)
    keep = ones != 0
    got, probs = eager.attend(q, k, v, None, None, None, None, types=[], att_span=1, use_relative=False,
                              dropout_keep=keep, dropout_p=p)
    scores = q @ k.transpose(-1, -2) / math.sqrt(D)
    want_p = torch.softmax(scores, -1) * ones
    assert torch.allclose(probs, want_p, rtol=1e-12, atol=1e-14)
    assert torch.allclose(got, want_p @ v, rtol=1e-12, atol=1e-14)
