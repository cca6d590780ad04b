"""bf16 corners beyond the 2e-2 absolute bound, held to the reference's own
bf16 numerics.

With few keys against many queries (Lk = 51, Lq = 429) and narrow log
buckets (32 buckets, max relative position 64), nearly every pair falls on
the saturated table rows, so one row of dKr sums some 65,000 terms of dS
times q that largely cancel, and the gradients of k, v and Qr are large.
There, bf16 rounding alone moves several gradients past 2e-2 absolute: the
reference's own op chain under bf16 autocast (its matmuls autocast to
bf16, deberta_v2_native.py:592-652; restated by running the oracle under
torch.autocast) lands 0.025 to 0.052 from the fp32 oracle on dk, dv, dKr
and dQr.  The kernels' own bf16 error there comes from bf16 dS and from
Delta = rowsum(dO * O) taken on the bf16 output (a per-row offset of dS
that the saturated row's sum does not cancel).  Both are held here to the
larger of the 2e-2 bound and 1.5x the reference's own bf16 error, tensor
by tensor, and the fp32 kernels to 1e-4 of scale on the same case.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import eager
from tests._cases import Case, hip_run, make_inputs, max_abs, max_rel, oracle_run

pytestmark = pytest.mark.gpu

CORNERS = [
    Case(B=3, H=3, L=429, D=64, buckets=32, max_pos=64, seed=70309, Lk=51),
    Case(B=2, H=2, L=700, D=64, buckets=16, max_pos=48, seed=70310, Lk=40),
]


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _reference_bf16(c: Case, x: dict) -> dict:
    """The oracle's op chain under CPU bf16 autocast on the bf16-rounded
    inputs (with the case's mask and dropout keep mask, as oracle_run
    gives them): the reference's own bf16 numerics."""
    types = c.type_list
    r = lambda t: t.to(torch.bfloat16).to(torch.float32).detach().clone().requires_grad_(True)
    q, k, v = (r(x[n]).permute(0, 2, 1, 3) for n in ("q", "k", "v"))
    kr = r(x["kr"]) if ("c2p" in types or "p2p" in types) else None
    qr = r(x["qr"]) if ("p2c" in types or "p2p" in types) else None
    use_rel = kr is not None or qr is not None
    Lk = c.Lk or c.L
    rel = eager.relative_positions(c.L, Lk, c.buckets, c.max_pos) if use_rel else None
    keep, p = None, 0.0
    if c.drop_t:
        from oracle.dropout import keep_mask

        keep = torch.from_numpy(keep_mask(c.drop_seed, c.drop_t, c.B, c.H, c.L, Lk))
        p = c.drop_t / 65536
    with torch.autocast("cpu", dtype=torch.bfloat16):
        ctx, _ = eager.attend(
            q, k, v, kr, qr, rel, x["mask"], types=types, att_span=c.A, use_relative=use_rel, dropout_keep=keep,
            dropout_p=p,
        )
    dout = x["dout"].to(torch.bfloat16).float().permute(0, 2, 1, 3)
    leaves = [t for t in (q, k, v, kr, qr) if t is not None]
    names = ["dq", "dk", "dv"] + (["dkr"] if kr is not None else []) + (["dqr"] if qr is not None else [])
    gs = torch.autograd.grad(ctx.float(), leaves, dout, allow_unused=True)
    res = {"out": ctx.float().permute(0, 2, 1, 3).detach()}
    for n, g, t in zip(names, gs, leaves):
        g = torch.zeros_like(t) if g is None else g.detach()
        res[n] = g.permute(0, 2, 1, 3) if n in ("dq", "dk", "dv") else g
    return res


@pytest.mark.parametrize("c", CORNERS, ids=str)
def test_bf16_corner_within_reference_bf16(c, gpu):
    x = make_inputs(c)
    exact = oracle_run(c, x, torch.bfloat16)
    ref16 = _reference_bf16(c, x)
    got = hip_run(c, x, torch.bfloat16, gpu)
    ours = {k: max_abs(got[k], exact[k]) for k in exact}
    theirs = {k: max_abs(ref16[k], exact[k]) for k in exact}
    _say(f"[bf16 corner] {c}\n  kernels {ours}\n  reference under autocast {theirs}")
    for k in exact:
        assert torch.isfinite(got[k]).all(), k
        assert ours[k] <= max(2e-2, 1.5 * theirs[k]), (k, ours[k], theirs[k])


@pytest.mark.parametrize("c", CORNERS, ids=str)
def test_fp32_corner_exact(c, gpu):
    x = make_inputs(c)
    exact = oracle_run(c, x, torch.float32)
    got = hip_run(c, x, torch.float32, gpu)
    errs = {k: max_rel(got[k], exact[k]) for k in exact}
    _say(f"[fp32 corner] {c} {errs}")
    assert all(e <= 1e-4 for e in errs.values()), errs
