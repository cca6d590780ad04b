"""Pins of the oracle's blocks around the attention (oracle/blocks.py) —
CPU only: each against the textbook formula it must equal, computed
independently in float64 (LayerNorm from its mean / variance definition,
GELU from the normal CDF via math.erf, BCE from the log-sigmoid form), and
the reference's own orderings and rules (residual added after the dense
layer, CLS context only without a pairwise mask, loss averaged over active
tokens with a floor of one)."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import blocks, eager

F64 = torch.float64


def _cfg(**kw):
    base = dict(hidden_size=16, intermediate_size=40, layer_norm_eps=1e-7, hidden_dropout_prob=0.0,
                position_buckets=8, max_relative_positions=16, max_position_embeddings=16)
    base.update(kw)
    return eager.make_config(**base)


def _ln64(x, w, b, eps):
    m = x.mean(-1, keepdim=True)
    v = ((x - m) ** 2).mean(-1, keepdim=True)
    return (x - m) / torch.sqrt(v + eps) * w + b


def _randomize(mod, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.randn(p.shape, generator=g, dtype=p.dtype) * 0.5)


def test_output_residual_norm_is_layernorm_of_dense_plus_residual():
    m = blocks.OutputResidualNorm(_cfg()).double().eval()
    _randomize(m, 0)
    g = torch.Generator().manual_seed(1)
    h, inp = torch.randn(2, 5, 16, generator=g, dtype=F64), torch.randn(2, 5, 16, generator=g, dtype=F64)
    z = h @ m.dense.weight.T + m.dense.bias + inp
    want = _ln64(z, m.LayerNorm.weight, m.LayerNorm.bias, 1e-7)
    torch.testing.assert_close(m(h, inp), want, rtol=0, atol=1e-12)


def test_intermediate_is_erf_gelu():
    m = blocks.Intermediate(_cfg()).double().eval()
    _randomize(m, 2)
    h = torch.randn(3, 16, generator=torch.Generator().manual_seed(3), dtype=F64)
    with torch.no_grad():
        z = h @ m.dense.weight.T + m.dense.bias
        want = z.clone().apply_(lambda t: 0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))))
        torch.testing.assert_close(m(h), want, rtol=0, atol=1e-12)


@torch.no_grad()
def test_rtd_head_cls_context_rule_and_order():
    m = blocks.RTDHead(_cfg()).double().eval()
    _randomize(m, 4)
    g = torch.Generator().manual_seed(5)
    h = torch.randn(2, 6, 16, generator=g, dtype=F64)
    gelu = lambda z: z.clone().apply_(lambda t: 0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))))
    def head(x):
        y = gelu(x @ m.dense.weight.T + m.dense.bias)
        return (y @ m.classifier.weight.T + m.classifier.bias).squeeze(-1)
    with_ctx = head(_ln64(h + h[:, :1], m.norm.weight, m.norm.bias, m.norm.eps))
    without = head(_ln64(h, m.norm.weight, m.norm.bias, m.norm.eps))
    torch.testing.assert_close(m(h), with_ctx, rtol=0, atol=1e-12)
    torch.testing.assert_close(m(h, torch.ones(2, 6, dtype=torch.bool)), with_ctx, rtol=0, atol=1e-12)
    torch.testing.assert_close(m(h, torch.ones(2, 1, 6, 6, dtype=torch.bool)), without, rtol=0, atol=1e-12)
    assert not torch.allclose(with_ctx, without)


def test_discriminator_loss_is_masked_mean_bce():
    g = torch.Generator().manual_seed(6)
    z = torch.randn(3, 7, generator=g, dtype=F64) * 4
    y = (torch.rand(3, 7, generator=g) < 0.3).to(F64)
    act = torch.rand(3, 7, generator=g) < 0.8
    per = -(y * torch.log(torch.sigmoid(z)) + (1 - y) * torch.log(torch.sigmoid(-z)))
    want = (per * act).sum() / act.sum()
    torch.testing.assert_close(blocks.discriminator_loss(z, y, act).double(), want, rtol=1e-6, atol=0)
    # no active token: the floor of one keeps it finite (zero)
    assert float(blocks.discriminator_loss(z, y, torch.zeros_like(act))) == 0.0


def test_relative_embeddings_layernorm():
    m = blocks.RelativeEmbeddings(_cfg()).double()
    _randomize(m, 7)
    assert m.rel_embeddings.weight.shape == (16, 16)  # 2 * buckets rows
    torch.testing.assert_close(m(), _ln64(m.rel_embeddings.weight, m.LayerNorm.weight, m.LayerNorm.bias, 1e-7),
                               rtol=0, atol=1e-12)
