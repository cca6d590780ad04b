"""The module under activation checkpointing (torch.utils.checkpoint).

The forward saves the relative term c2p + p2c for the backward, an (L, L)
tensor per (batch row, head), 2 bytes an element in bf16.  Checkpointing is
how a caller keeps it from living across layers: reentrant checkpointing
runs the first forward without gradients, so the term is not written at all,
and non-reentrant checkpointing drops the forward's saved tensors and
recomputes them in the backward.  Both must give the plain module's output
and gradients (the relative-table gradients up to the order of their fp32
atomic additions), and the memory held between forward and backward must
drop by at least the saved term.
"""

from __future__ import annotations

import sys

import pytest
import torch
import torch.utils.checkpoint as ckpt

from deberta_amd import DisentangledSelfAttention
from oracle import eager
from tests._cases import max_rel

pytestmark = pytest.mark.gpu

B, L, HIDDEN, HEADS = 8, 512, 256, 4


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _module(gpu):
    cfg = eager.make_config(
        hidden_size=HIDDEN, num_attention_heads=HEADS, position_buckets=256, max_relative_positions=512,
        share_att_key=True,
    )
    torch.manual_seed(0)
    m = DisentangledSelfAttention(cfg)
    with torch.no_grad():
        for n, p in m.named_parameters():
            p.copy_(torch.randn_like(p) * 0.02 if n.endswith("weight") else torch.zeros_like(p))
    return m.to(gpu).eval()


def _inputs(gpu):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, L, HIDDEN, generator=g).to(gpu).requires_grad_(True)
    rel = (torch.randn(512, HIDDEN, generator=g) * 0.02).to(gpu).requires_grad_(True)
    dout = torch.randn(B, L, HIDDEN, generator=g).to(gpu)
    return x, rel, dout


def _step(module, mode, gpu):
    """Forward (bf16 autocast) in one of three modes, the memory held after
    it, then the backward: (out, {name: grad}, bytes held)."""
    x, rel, dout = _inputs(gpu)
    params = list(module.named_parameters())

    def fwd(x_, rel_):
        return module(x_, None, rel_embeddings=rel_)[0]

    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        if mode == "plain":
            out = fwd(x, rel)
        else:
            out = ckpt.checkpoint(fwd, x, rel, use_reentrant=(mode == "reentrant"))
    torch.cuda.synchronize()
    held = torch.cuda.memory_allocated(gpu) - base
    # .backward() (reentrant checkpointing does not support autograd.grad)
    for _, p in params:
        p.grad = None
    out.backward(dout.to(out.dtype))
    grads = {"x": x.grad.float(), "rel": rel.grad.float()}
    grads.update({n: p.grad.float() for n, p in params})
    return out.detach().float(), grads, held


# Gradients that pass through the relative tables' fp32 atomics: their
# sums vary in the last fp32 bits from run to run and are written in the
# tables' dtype, bf16 under autocast, where such a difference can round to
# the neighbouring value (2^-8 relative); held to two bf16 steps of their
# scale.
_ATOMIC = ("rel", "key_proj.weight", "key_proj.bias", "query_proj.weight", "query_proj.bias")
_ATOMIC_TOL = 2.0**-7


@pytest.mark.parametrize("mode", ["reentrant", "non_reentrant"])
def test_checkpointed_module_matches_plain(mode, gpu):
    module = _module(gpu)
    out0, g0, held0 = _step(module, "plain", gpu)
    out1, g1, held1 = _step(module, mode, gpu)
    saved_term = B * HEADS * L * L * 2  # fp16 relative term the plain forward keeps
    errs = {n: max_rel(g1[n], g0[n]) for n in g0}
    _say(f"[checkpoint {mode}] held {held0 / 2**20:.1f} -> {held1 / 2**20:.1f} MiB "
         f"(saved term {saved_term / 2**20:.1f} MiB); worst grads "
         f"{sorted(errs.items(), key=lambda kv: -kv[1])[:3]}")
    assert torch.equal(out1, out0)
    assert torch.equal(g1["x"], g0["x"]), "dx differs (no atomics on its path)"
    for n in g0:
        if n.endswith("key_proj.bias"):
            continue  # exact gradient zero (a shift of every key): rounding noise only
        tol = _ATOMIC_TOL if any(n.endswith(a) for a in _ATOMIC) else 0.0
        assert errs[n] <= tol, (n, errs[n])
    assert held0 - held1 >= saved_term, (held0, held1, saved_term)
