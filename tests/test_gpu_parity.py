"""Parity of the HIP kernels (through the custom-op boundary) with the CPU
oracle, on identical seeded inputs.

Tolerances:
  bf16: max |hip - oracle| <= 2e-2 on the output and every gradient, with the
        oracle in fp32 on the bf16-rounded inputs;
  fp32: max |hip - oracle| / max |oracle| <= 1e-4 on the output and every
        gradient.
"""

from __future__ import annotations

import sys

import pytest
import torch

from tests._cases import Case, hip_run, make_inputs, max_abs, max_rel, oracle_run

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2
FP32_TOL = 1e-4


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _check(c: Case, dtype: torch.dtype, gpu, grads: bool = True, zero: tuple = (), grads_to_scale: bool = False) -> dict:
    """``zero``: tensors whose exact value is zero (both sides hold rounding
    noise only), held to the tolerance absolutely.  ``grads_to_scale``: bf16
    gradients held to the tolerance relative to their scale (max|err| /
    max|ref|) instead of absolutely."""
    _say(f"[parity] {c} dtype={dtype}")
    x = make_inputs(c)
    ref = oracle_run(c, x, dtype, grads)
    got = hip_run(c, x, dtype, gpu, grads)
    errs = {}
    for name, r in ref.items():
        g = got[name]
        assert g.shape == r.shape, (name, g.shape, r.shape)
        assert torch.isfinite(g).all(), f"{name} has non-finite values"
        absolute = (dtype == torch.bfloat16 and not (grads_to_scale and name.startswith("d"))) or name in zero
        errs[name] = max_abs(g, r) if absolute else max_rel(g, r)
    _say(f"[parity]   errors {errs}")
    tol = BF16_TOL if dtype == torch.bfloat16 else FP32_TOL
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, f"{c}: {bad} exceed {tol}"
    return got


# --- forward + backward, no mask -------------------------------------------------
@pytest.mark.parametrize(
    "c",
    [
        Case(B=2, H=12, L=512, D=64),  # config-2 shape, 2 batch rows
        Case(B=32, H=12, L=512, D=64, seed=9),  # the benchmark's full shape (B=32)
        Case(B=1, H=2, L=200, D=64, seed=1),  # ragged tiles
        Case(B=2, H=3, L=130, D=64, types="c2p", seed=2),
        Case(B=2, H=3, L=130, D=64, types="p2c", seed=3),
        Case(B=2, H=3, L=130, D=64, types="", seed=4),
        Case(B=1, H=2, L=256, D=32, seed=5),
    ],
    ids=str,
)
def test_bf16_no_mask(c, gpu):
    _check(c, torch.bfloat16, gpu)


@pytest.mark.parametrize(
    "c",
    [
        Case(B=2, H=4, L=128, D=32, seed=0),  # config-1 shape
        Case(B=1, H=2, L=300, D=64, seed=6),
        Case(B=1, H=2, L=96, D=64, types="p2c", seed=7),
    ],
    ids=str,
)
def test_fp32_no_mask(c, gpu):
    _check(c, torch.float32, gpu)


# --- masks --------------------------------------------------------------------------
# --- growing scores: the forward's reference max is raised on most key tiles ----
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("mask", ["none", "key"])
def test_growing_scores(mask, dtype, gpu):
    """Keys scaled up along the sequence, so each 64-key tile's score maxima
    exceed the previous ones by far more than the forward's reference-max
    slack (8 in log2 units): the running max is raised and O and l rescaled
    tile after tile, and softmax rows are nearly one-hot."""
    if dtype == torch.float32:
        c = Case(B=2, H=2, L=384, D=64, std=2.0, ramp=3.0, mask=mask, seed=41)  # log2 scores to +-50
        _check(c, dtype, gpu)
    else:
        # Scores to +-28 (log2 units): larger ones put the fp16-stored relative
        # term's rounding (2^-10 relative) above the absolute bf16 tolerance,
        # as the reference's own bf16 products (2^-9) would be.  Gradients at
        # these magnitudes are large (the keys are scaled up to 9x), so they
        # are held to the tolerance relative to their scale.
        c = Case(B=2, H=2, L=384, D=64, std=1.0, ramp=8.0, mask=mask, seed=41)
        _check(c, dtype, gpu, grads_to_scale=True)


# --- long sequences (config-4 length, with its document-block mask) and the
# config-5 head count: 32 query tiles, 64 offset blocks, the ring of qrgt
# blocks wrapping many times, tile skipping over whole documents
@pytest.mark.parametrize(
    "c,dtype",
    [
        (Case(B=1, H=2, L=4096, D=64, mask="pair", seed=51), torch.bfloat16),
        (Case(B=1, H=2, L=4096, D=64, mask="pair", seed=52), torch.float32),
        (Case(B=1, H=2, L=4096, D=64, mask="seg", seed=51), torch.bfloat16),
        (Case(B=1, H=2, L=4096, D=64, mask="seg", seed=52), torch.float32),
        (Case(B=1, H=2, L=4096, D=64, seed=53), torch.bfloat16),
        (Case(B=2, H=2, L=2048, D=64, mask="key", seed=54), torch.float32),
        (Case(B=2, H=16, L=512, D=64, seed=55), torch.bfloat16),
    ],
    ids=["L4096-doc-bf16", "L4096-doc-fp32", "L4096-seg-bf16", "L4096-seg-fp32", "L4096-bf16", "L2048-key-fp32", "H16-bf16"],
)
def test_long_sequences(c, dtype, gpu):
    _check(c, dtype, gpu)


# --- short sequences: the reference's own tests run 4 and 8 tokens
# (tests/test_smoke.py:1875, 1951, 2015, 2054, 1794); every tile is mostly
# padding and the relative table has 2L - 1 entries
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize(
    "c",
    [
        Case(B=2, H=4, L=1, D=32, seed=71),
        Case(B=2, H=4, L=4, D=32, seed=72),
        Case(B=2, H=4, L=8, D=64, seed=73),
        Case(B=2, H=4, L=8, D=64, mask="key", seed=74),
        Case(B=3, H=2, L=17, D=64, mask="seg", seed=75),
        Case(B=2, H=2, L=33, D=64, mask="pair", seed=76),
        Case(B=2, H=2, L=63, D=32, types="p2c", seed=77),
        Case(B=1, H=2, L=4, D=64, Lk=8, seed=78),
    ],
    ids=str,
)
def test_short_sequences(c, dtype, gpu):
    # one key: the softmax is constant (P = 1), so the score gradient dS and
    # with it dq, dk, dkr, dqr are exactly zero
    one_key = (c.Lk or c.L) == 1
    _check(c, dtype, gpu, zero=("dq", "dk", "dkr", "dqr") if one_key else ())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("mask", ["key", "pair", "pair_auto", "seg", "seg_mixed", "dead"])
def test_masks(mask, dtype, gpu):
    c = Case(B=3, H=2, L=260, D=64, mask=mask, seed=11)
    got = _check(c, dtype, gpu)
    x = make_inputs(c)
    m = x["mask"][:, 0]
    live = m[:, 0, :] if m.shape[1] == 1 else torch.diagonal(m, dim1=-2, dim2=-1)
    dead = ~live
    if dead.any():
        # dead query rows: output exactly zero, no gradient into q
        assert float(got["out"][dead].abs().max()) == 0.0
        assert float(got["dq"][dead].abs().max()) == 0.0


def test_document_mask_runs_as_segments(gpu):
    """A dense packed-document mask is recognised and run as segment ids:
    the results equal those of the dense pair-mask kernels bit for bit
    (skipped tiles only ever add exact zeros), dKr / dQr up to the order of
    their fp32 atomic additions."""
    import dataclasses

    c = Case(B=2, H=2, L=384, D=64, mask="pair", seed=61)
    x = make_inputs(c)
    dense = hip_run(c, x, torch.bfloat16, gpu)
    auto = hip_run(dataclasses.replace(c, mask="pair_auto"), x, torch.bfloat16, gpu)
    print(f"[doc mask as segments] keys {sorted(dense)}", file=sys.stderr, flush=True)
    for name in ("out", "lse", "dq", "dk", "dv"):
        assert torch.equal(dense[name], auto[name]), name
    for name in ("dkr", "dqr"):
        assert max_rel(auto[name], dense[name]) <= 1e-2, name


# --- relative-position configurations --------------------------------------------
@pytest.mark.parametrize(
    "c",
    [
        # no bucketing: A = max_relative_positions = 512, 1024 table rows
        Case(B=1, H=2, L=300, D=64, buckets=-1, max_pos=512, seed=21),
        # small buckets: long saturated tails
        Case(B=1, H=2, L=300, D=64, buckets=32, max_pos=64, seed=22),
        # a log base close to 0: bucket jumps of many rows per offset (band chunking)
        Case(B=1, H=2, L=300, D=64, buckets=256, max_pos=130, seed=23),
        # sequence longer than max_position: saturation both ways
        Case(B=1, H=1, L=700, D=64, buckets=256, max_pos=512, seed=24),
    ],
    ids=str,
)
def test_relative_configs(c, gpu):
    _check(c, torch.bfloat16, gpu)


def test_relative_configs_fp32(gpu):
    _check(Case(B=1, H=2, L=300, D=32, buckets=32, max_pos=64, seed=25), torch.float32, gpu)


# --- determinism of the forward (recompute under gradient checkpointing) ------------
def test_forward_is_deterministic(gpu):
    c = Case(B=2, H=4, L=256, D=64, mask="key", seed=31)
    x = make_inputs(c)
    a = hip_run(c, x, torch.bfloat16, gpu, grads=False)
    b = hip_run(c, x, torch.bfloat16, gpu, grads=False)
    assert torch.equal(a["out"], b["out"]) and torch.equal(a["lse"], b["lse"])
