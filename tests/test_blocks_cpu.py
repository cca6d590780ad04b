"""The fused blocks on CPU tensors: each runs the reference's block in torch
operations there (the row kernels run on the GPU only), held to the
oracle's restatement (``oracle/blocks.py``) with identical weights: output
and every input and parameter gradient, fp32, max|err| / max|ref| <= 1e-5
per tensor.  Hidden dropout in training acts on the dense output with its
bias, as the reference's ``dropout(dense(x))``: with one seed both draw the
same mask."""

from __future__ import annotations

import pytest
import torch

from deberta_amd import FusedIntermediate, FusedOutput, FusedRTDHead, FusedSelfOutput, RelativeEmbeddings
from oracle import blocks as ob
from oracle import eager
from tests._cases import max_rel

TOL = 1e-5


def _cfg(**kw):
    return eager.make_config(hidden_size=64, num_attention_heads=4, intermediate_size=192, layer_norm_eps=1e-7, **kw)


def _same(ours, ref, seed=0):
    torch.manual_seed(seed)
    with torch.no_grad():
        for p in ref.parameters():
            p.copy_(torch.randn_like(p) * 0.3)
    ours.load_state_dict(ref.state_dict(), strict=True)
    return ours, ref


def _grads(module, inputs, extra=None):
    leaves = [t.detach().clone().requires_grad_(t.is_floating_point()) for t in inputs]
    out = module(*leaves) if extra is None else extra(module, leaves)
    if isinstance(out, tuple):
        out = out[0]
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(1)) if out.dim() else torch.ones(())
    wrt = [t for t in leaves if t.requires_grad] + list(module.parameters())
    grads = torch.autograd.grad(out, wrt, g, allow_unused=True)
    return [out.detach()] + [torch.zeros(1) if x is None else x for x in grads]


def _compare(a, b):
    errs = [max_rel(x, y) for x, y in zip(b, a)]
    assert all(e <= TOL for e in errs), errs


@pytest.mark.parametrize("kind", ["self_output", "output"])
def test_output_blocks_on_cpu(kind):
    cfg = _cfg()
    width = 64 if kind == "self_output" else 192
    ours = FusedSelfOutput(cfg) if kind == "self_output" else FusedOutput(cfg)
    ours, ref = _same(ours, ob.OutputResidualNorm(cfg, in_features=width))
    g = torch.Generator().manual_seed(3)
    x, res = torch.randn(2, 10, width, generator=g), torch.randn(2, 10, 64, generator=g)
    _compare(_grads(ref.eval(), [x, res]), _grads(ours.eval(), [x, res]))


def test_intermediate_relative_embeddings_and_head_on_cpu():
    cfg = _cfg()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 10, 64, generator=g)
    ours, ref = _same(FusedIntermediate(cfg), ob.Intermediate(cfg))
    _compare(_grads(ref, [x]), _grads(ours, [x]))
    ours, ref = _same(RelativeEmbeddings(cfg), ob.RelativeEmbeddings(cfg))
    _compare(_grads(ref, []), _grads(ours, []))
    ours, ref = _same(FusedRTDHead(cfg), ob.RTDHead(cfg))
    for mask in (None, torch.ones(2, 1, 10, 10, dtype=torch.bool)):
        _compare(
            _grads(ref, [x], lambda m, l: m(l[0], attention_mask=mask)),
            _grads(ours, [x], lambda m, l: m(l[0], attention_mask=mask)),
        )
    labels = (torch.rand(2, 10, generator=g) < 0.15).float()
    active = torch.ones(2, 10, dtype=torch.bool)
    active[1, 7:] = False

    def ref_loss(m, l):
        return ob.discriminator_loss(m(l[0]), labels, active)

    def our_loss(m, l):
        return m.forward_loss(l[0], labels, active)[0]

    _compare(_grads(ref, [x], ref_loss), _grads(ours, [x], our_loss))


def test_hidden_dropout_on_cpu_matches_the_reference_block():
    cfg = _cfg(hidden_dropout_prob=0.25)
    ours, ref = _same(FusedSelfOutput(cfg), ob.OutputResidualNorm(cfg))
    g = torch.Generator().manual_seed(6)
    x, res = torch.randn(2, 10, 64, generator=g), torch.randn(2, 10, 64, generator=g)
    ours.train(), ref.train()
    torch.manual_seed(11)
    a = ref(x, res)
    torch.manual_seed(11)
    b = ours(x, res)
    assert max_rel(b, a) <= TOL
    torch.manual_seed(12)
    assert max_rel(ours(x, res), a) > 1e-3  # another mask
