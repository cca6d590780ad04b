"""A seeded matrix of op-level parity cases on the GPU: combinations of
element type, head dim, relative terms, bucketing, mask form, dropout and
ragged extents that the targeted cases in test_gpu_parity.py take one at a
time.  The list is drawn once, from a fixed CPU generator, so every run
checks the same cases; each is held to test_gpu_parity.py's bar against
the CPU oracle (bf16: 2e-2 absolute; fp32: 1e-4 of max|ref|)."""

from __future__ import annotations

import pytest
import torch

from tests._cases import Case
from tests.test_gpu_parity import _check

pytestmark = pytest.mark.gpu

_TYPES = ["c2p|p2c", "c2p|p2c", "c2p", "p2c", ""]
_BUCKETS = [(256, 512), (32, 64), (-1, 64), (128, 256), (64, 512)]
_MASKS = ["none", "none", "key", "pair", "pair_auto", "seg", "seg_mixed", "dead"]


def _draw(n: int, seed: int = 2024) -> list[tuple[Case, torch.dtype]]:
    g = torch.Generator().manual_seed(seed)
    pick = lambda seq: seq[int(torch.randint(len(seq), (1,), generator=g))]
    cases = []
    for i in range(n):
        dtype = torch.bfloat16 if i % 2 == 0 else torch.float32
        buckets, max_pos = pick(_BUCKETS)
        mask = pick(_MASKS)
        L = int(torch.randint(16, 701, (1,), generator=g))
        # masks need Lq == Lk; unmasked cases may have Lk != Lq
        Lk = None
        if mask == "none" and int(torch.randint(3, (1,), generator=g)) == 0:
            Lk = int(torch.randint(16, 701, (1,), generator=g))
        dropout = 0.1 if int(torch.randint(4, (1,), generator=g)) == 0 else 0.0
        c = Case(
            B=int(torch.randint(1, 4, (1,), generator=g)),
            H=int(torch.randint(1, 5, (1,), generator=g)),
            L=L,
            D=pick([32, 64]),
            buckets=buckets,
            max_pos=max_pos,
            types=pick(_TYPES),
            mask=mask,
            seed=100 + i,
            Lk=Lk,
            dropout=dropout,
        )
        cases.append((c, dtype))
    return cases


_CASES = _draw(96)


@pytest.mark.parametrize(
    "c,dtype", _CASES, ids=[f"{i}-{'bf16' if d == torch.bfloat16 else 'fp32'}" for i, (_, d) in enumerate(_CASES)]
)
def test_matrix_case(c, dtype, gpu):
    _check(c, dtype, gpu)
