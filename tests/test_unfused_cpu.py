"""CPU parity of ``deberta_amd.unfused.unfused_attention`` (the module's
torch-operation path for output_attentions, attention dropout and
non-Toeplitz relative positions) against the oracle's ``attend``: context,
probabilities and every input gradient, fp32, on identical inputs.

The path is torch device operations only, so the CPU runs it as the GPU
does; the GPU module tests (tests/test_gpu_unfused.py) cover its wiring in
``DisentangledSelfAttention``.  Tolerance: max|err| / max|ref| <= 1e-5 per
tensor (both sides fp32, differing in operation order only).
"""

from __future__ import annotations

import math

import pytest
import torch

from deberta_amd.unfused import unfused_attention
from oracle import eager
from tests._cases import max_rel


def _case(types, mask, rel_kind, B=2, L=40, H=3, D=16, A=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, L, H, D, generator=g) for _ in range(3))
    kr, qr = torch.randn(H, 2 * A, D, generator=g), torch.randn(H, 2 * A, D, generator=g)
    if rel_kind == "canonical":
        rel = eager.relative_positions(L, L, 4, 16)
    else:  # not a function of i - j: arbitrary ids, beyond the span too
        rel = torch.randint(-2 * A, 2 * A + 1, (L, L), generator=g)
    keep = None
    if mask == "padding":
        km = torch.ones(B, L, dtype=torch.bool)
        km[1, 29:] = False
        keep = km[:, None, None, :]
    elif mask == "pair":
        keep = torch.rand(B, 1, L, L, generator=g) < 0.7
        keep[0, 0, 5, :] = False  # a dead query row
        keep[0, 0, 5, 0] = True
        keep[0, 0, 5, 5] = False
    elif mask == "per_head":
        keep = torch.rand(B, H, L, L, generator=g) < 0.6
        keep |= torch.eye(L, dtype=torch.bool)
        keep[1, 2, 7, 7] = False  # dead in one head only
    return q, k, v, kr, qr, rel, keep, A


@pytest.mark.parametrize("types", ["c2p|p2c", "c2p|p2c|p2p", "p2c", "c2p", "p2p", "none"])
@pytest.mark.parametrize("mask", ["none", "padding", "pair", "per_head"])
@pytest.mark.parametrize("rel_kind", ["canonical", "arbitrary"])
def test_unfused_matches_oracle(types, mask, rel_kind):
    tl = eager.pos_att_types(types if types != "none" else None)
    q, k, v, kr, qr, rel, keep, A = _case(tl, mask, rel_kind)
    sf = 1 + sum(t in tl for t in ("c2p", "p2c", "p2p"))
    scale = 1.0 / math.sqrt(q.shape[-1] * sf)
    use_rel = bool(tl)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, kr, qr)]
    ctx, probs = unfused_attention(*leaves[:5], rel if use_rel else None, keep, A, scale, tl)
    ref_leaves = [t.clone().requires_grad_(True) for t in (q, k, v, kr, qr)]
    rq, rk, rv = (t.permute(0, 2, 1, 3) for t in ref_leaves[:3])
    rctx, rprobs = eager.attend(rq, rk, rv, ref_leaves[3], ref_leaves[4], rel, keep, types=tl, att_span=A,
                                use_relative=use_rel)
    rctx = rctx.permute(0, 2, 1, 3)
    assert max_rel(ctx, rctx) <= 1e-5
    assert max_rel(probs, rprobs) <= 1e-5
    dout = torch.randn(ctx.shape, generator=torch.Generator().manual_seed(9))
    got = torch.autograd.grad(ctx, leaves, dout, allow_unused=True)
    want = torch.autograd.grad(rctx, ref_leaves, dout, allow_unused=True)
    for name, a, b in zip(("dq", "dk", "dv", "dkr", "dqr"), got, want):
        if b is None:
            assert a is None or float(a.abs().max()) == 0.0, name
            continue
        assert max_rel(a, b) <= 1e-5, name


def test_unfused_dropout_acts_on_the_probabilities():
    """Dropout is applied after the softmax (and before the dead-row zeroing):
    the kept probabilities are the plain ones over (1 - p), the context is
    the dropped probabilities times v."""
    q, k, v, kr, qr, rel, keep, A = _case(["c2p", "p2c"], "padding", "canonical", L=64)
    scale = 1.0 / math.sqrt(q.shape[-1] * 3)
    torch.manual_seed(5)
    drop = torch.nn.Dropout(0.25).train()
    ctx, probs = unfused_attention(q, k, v, kr, qr, rel, keep, A, scale, ["c2p", "p2c"], drop)
    _, plain = unfused_attention(q, k, v, kr, qr, rel, keep, A, scale, ["c2p", "p2c"])
    kept = probs != 0
    pos = plain != 0
    frac = 1.0 - float(kept[pos].float().mean())
    assert 0.2 < frac < 0.3, frac
    assert torch.allclose(probs[kept], plain[kept] / 0.75, rtol=1e-6, atol=0)
    want = torch.matmul(probs, v.permute(0, 2, 1, 3)).permute(0, 2, 1, 3)
    assert max_rel(ctx, want) <= 1e-6
