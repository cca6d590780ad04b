"""Pins of the relative-position oracle (oracle/eager.py: log_bucket,
relative_positions) and of the product's host-side copies
(deberta_amd/relpos.py).

The reference holds no known-answer vectors for the bucket function; it is
pinned here by its closed form evaluated in double precision
(oracle/brute.py: bucket_exact), by the invariants the published formula
fixes, and by the reference's own saturation test (test_smoke.py:2225).
"""

from __future__ import annotations

import pytest
import torch

from deberta_amd import relpos
from oracle import brute, eager

CONFIGS = [(256, 512), (128, 512), (32, 64), (8, 16), (512, 1024)]


@pytest.mark.parametrize("bs,mp", CONFIGS)
def test_identity_below_mid(bs, mp):
    mid = bs // 2
    d = torch.arange(-(mid - 1), mid)
    assert torch.equal(eager.log_bucket(d, bs, mp), d)


@pytest.mark.parametrize("bs,mp", CONFIGS)
def test_odd_symmetry_and_mid(bs, mp):
    d = torch.arange(0, 4 * mp)
    pos = eager.log_bucket(d, bs, mp)
    neg = eager.log_bucket(-d, bs, mp)
    assert torch.equal(neg, -pos)
    mid = bs // 2
    assert int(eager.log_bucket(torch.tensor([mid]), bs, mp)) == mid


@pytest.mark.parametrize("bs,mp", CONFIGS)
def test_monotone_unit_steps(bs, mp):
    """Non-decreasing in d with steps of 0 or 1: the property the kernels'
    contiguous per-row offset ranges rely on."""
    d = torch.arange(-4 * mp, 4 * mp + 1)
    b = eager.log_bucket(d, bs, mp)
    steps = b[1:] - b[:-1]
    assert bool(((steps == 0) | (steps == 1)).all())


def test_saturation_reference_case():
    """test_smoke.py:2225 restated: with bucket_size=128, max_position=512
    every |d| >= 511 maps to the bucket of +-511."""
    d = torch.tensor([-999, -800, -511, -510, 0, 510, 511, 800, 999])
    b = eager.log_bucket(d, 128, 512)
    assert b[0] == b[2] and b[1] == b[2]
    assert b[-1] == b[6] and b[-2] == b[6]


def test_saturation_value_256_512():
    """Saturated offsets land on +-(2*mid - 1) = +-255 (the fp32 ratio at
    |d| = max_position - 1 is exactly mid - 1 before ceil)."""
    d = torch.tensor([511, 600, 4095, -511, -4095])
    assert eager.log_bucket(d, 256, 512).tolist() == [255, 255, 255, -255, -255]


def test_all_buckets_hit_256_512():
    d = torch.arange(128, 512)
    vals = set(eager.log_bucket(d, 256, 512).tolist())
    assert vals == set(range(128, 256))


@pytest.mark.parametrize("bs,mp", [(256, 512), (128, 512), (32, 64)])
def test_matches_double_precision_closed_form(bs, mp):
    """fp32 evaluation (the reference's) equals the double-precision closed
    form except where the pre-ceil value is within 1e-4 of an integer; those
    points are only |d| = mid (value 0) and the saturation edge."""
    span = range(-2 * mp, 2 * mp + 1)
    got = eager.log_bucket(torch.tensor(list(span)), bs, mp).tolist()
    mid = bs // 2
    near = []
    for d, g in zip(span, got):
        exact, ambiguous = brute.bucket_exact(d, bs, mp)
        if ambiguous:
            near.append(abs(d))
            continue
        assert g == exact, (d, g, exact)
    assert set(near) <= {mid} | set(range(mp - 1, 2 * mp + 1))


def test_plain_relative_positions():
    rel = eager.relative_positions(5, 7, -1, 512)
    assert rel[2, 4] == -2 and rel[4, 0] == 4
    assert torch.equal(rel, torch.arange(5)[:, None] - torch.arange(7)[None, :])


# --- the product's host-side helpers agree with the oracle -----------------------
@pytest.mark.parametrize("bs,mp", CONFIGS + [(-1, 512)])
@pytest.mark.parametrize("lq,lk", [(8, 8), (130, 130), (600, 600), (5, 9)])
def test_product_relpos_matches_oracle(bs, mp, lq, lk):
    ref = eager.relative_positions(lq, lk, bs, mp)
    got = relpos.build_relative_position(lq, lk, bucket_size=bs, max_position=mp)
    assert torch.equal(got, ref)
    table = relpos.relative_offset_table(lq, lk, bucket_size=bs, max_position=mp)
    idx = torch.arange(lq)[:, None] - torch.arange(lk)[None, :] + (lk - 1)
    assert torch.equal(table.long()[idx], ref)
    assert torch.equal(relpos.table_from_matrix(ref), table)
    assert relpos.is_toeplitz(ref)
    assert relpos.is_monotone(table)


def test_is_toeplitz_rejects_other_matrices():
    rel = eager.relative_positions(16, 16, 8, 16).clone()
    rel[3, 7] += 1
    assert not relpos.is_toeplitz(rel)
    flipped = -eager.relative_positions(16, 16, 8, 16)
    assert relpos.is_toeplitz(flipped) and not relpos.is_monotone(relpos.table_from_matrix(flipped))


def test_normalize_relative_pos_ranks():
    rel = eager.relative_positions(6, 6, -1, 16)
    for shaped in (rel, rel[None], rel[None, None]):
        assert torch.equal(relpos.normalize_relative_pos(shaped, 4, 5), rel[:4, :5])
    with pytest.raises(ValueError, match="rank-2/3/4"):
        relpos.normalize_relative_pos(rel[None, None, None], 6, 6)


def test_log_base_nonpositive_is_identity():
    d = torch.arange(-40, 41)
    # max_position - 1 <= mid makes the log base log((mid+1)/mid) > 0; a
    # bucket size of 2 has mid = 1 -> identity (deberta_v2_native.py:70-71)
    assert torch.equal(eager.log_bucket(d, 2, 64), d.clamp(-63, 63))
