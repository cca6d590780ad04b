"""BASELINE configurations 3 and 5 as stated, on the GPU.

C5: one DeBERTa-v3-large-shaped attention layer (hidden 1024, 16 heads x
64, L = 512, c2p|p2c, buckets 256 / max relative positions 512, full mask)
run inside ``torch.compile`` under bf16 autocast, so the ops go through
their fake implementations.  At B = 2 it is compared with the fp32 oracle
module; at the full B = 64 the compiled layer is compared with the same
layer run eagerly.

C3: the 12-layer encoder harness (tests/_encoder.py) with the fused module
in every layer and the fused row kernels around it.  At B = 2 in fp32 it is
compared with the same encoder built on the oracle module and plain torch
blocks on the CPU (identical weights, ids and labels);
at the full B = 16 under bf16 autocast it is compared with the same encoder
whose attention runs on its torch-operation path.

Tolerances: fp32 max|err| / max|ref| <= 1e-4 per tensor.  bf16: the
layer's output and input gradient max|err| <= 2e-2 against the fp32 oracle
(the north_star's bound); the parameter gradients, which sum over B x L
rows and so exceed the resolution of bf16 at their own magnitude, max|err|
<= 2e-2 x max|ref| (relative to their scale).
"""

from __future__ import annotations

import sys

import pytest
import torch

from deberta_amd import DisentangledSelfAttention
from oracle import eager
from tests import _encoder
from tests._cases import max_abs, max_rel
from tests._modules import _errors, _pair, _run

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _c5_config():
    return eager.make_config(hidden_size=1024, num_attention_heads=16, share_att_key=True,
                             pos_att_type="p2c|c2p", position_buckets=256, max_relative_positions=512)


def test_c5_compiled_layer_against_oracle(gpu):
    """C5 layer, B = 2, torch.compile (inductor) + bf16 autocast, against
    the fp32 oracle module on the CPU with the same weights."""
    torch._dynamo.reset()
    ref, ours = _pair(_c5_config(), seed=5)
    ours = ours.to(gpu)
    compiled = torch.compile(ours, backend="inductor", dynamic=False)
    g = torch.Generator().manual_seed(55)
    x = torch.randn(2, 512, 1024, generator=g)
    rel = torch.randn(512, 1024, generator=g)
    a = _run(ref, x, None, rel, "cpu")
    b = _run(compiled, x, None, rel, gpu, autocast=True)
    errs = _errors(a, b)
    abs_errs = {k: max_abs(b[k], a[k]) for k in ("out", "dx")}
    _say(f"[C5 compiled B=2] abs {abs_errs} rel-to-scale {errs}")
    assert all(e <= 2e-2 for e in abs_errs.values()), abs_errs
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_c5_compiled_full_size_equals_eager(gpu):
    """C5 at its full size (B = 64): the compiled layer's output and
    gradients equal the eager layer's (the same kernels, reached through the
    fake implementations) and are finite."""
    torch._dynamo.reset()
    torch.manual_seed(0)
    layer = DisentangledSelfAttention(_c5_config()).to(gpu)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            p.copy_(torch.randn_like(p) * 0.02 if n.endswith("weight") else torch.zeros_like(p))
    g = torch.Generator().manual_seed(56)
    x = torch.randn(64, 512, 1024, generator=g).to(gpu)
    rel = (torch.randn(512, 1024, generator=g) * 0.02).to(gpu)
    compiled = torch.compile(layer, backend="inductor", dynamic=False)
    a = _run(layer, x, None, rel, gpu, autocast=True)
    b = _run(compiled, x, None, rel, gpu, autocast=True)
    for k in a:
        assert torch.isfinite(b[k]).all(), k
    errs = {k: max_rel(b[k], a[k]) for k in a}
    _say(f"[C5 compiled B=64 vs eager] {errs}")
    assert all(e <= 2e-2 for e in errs.values()), errs


def _encoder_pair(layers):
    """The oracle encoder (oracle attention, plain torch blocks) and the
    fused one (fused attention and fused row kernels), same weights."""
    ref = _encoder.Encoder(eager.EagerDisentangledSelfAttention, layers=layers)
    _encoder.init_weights(ref, seed=3)
    ours = _encoder.Encoder(DisentangledSelfAttention, layers=layers, fused_blocks=True)
    ours.load_state_dict(ref.state_dict(), strict=True)
    return ref, ours


def _encoder_step(model, ids, labels, rel_pos, mask, autocast=False):
    dev = ids.device
    with torch.autocast(dev.type, dtype=torch.bfloat16, enabled=autocast):
        loss, logits = model.loss(ids, mask, rel_pos, labels)
    names = [n for n, _ in model.named_parameters()]
    grads = torch.autograd.grad(loss, [p for _, p in model.named_parameters()])
    return logits.detach().float().cpu(), loss.detach().float().cpu(), {n: g.float().cpu() for n, g in zip(names, grads)}


def test_c3_encoder_fp32_against_oracle(gpu):
    """C3 encoder (12 layers), B = 2, fp32: the fused attention and fused
    blocks against the oracle attention and plain torch blocks, logits,
    loss and every parameter gradient."""
    ref, ours = _encoder_pair(_encoder.LAYERS)
    ours = ours.to(gpu)
    ids, labels = _encoder.synthetic_batch(2, 512, seed=1)
    mask = torch.ones(2, 1, 1, 512, dtype=torch.bool)
    rp_c = eager.relative_positions(512, 512, _encoder.BUCKETS, _encoder.MAX_POS)
    la, sa, ga = _encoder_step(ref, ids, labels, rp_c, mask)
    lb, sb, gb = _encoder_step(ours, ids.to(gpu), labels.to(gpu), rp_c.to(gpu), mask.to(gpu))
    errs = {"logits": max_rel(lb, la), "loss": max_rel(sb, sa)}
    for n in ga:
        if n.endswith("self.key_proj.bias"):
            # mostly cancelling (a shift of every key is a per-row constant
            # in the content and c2p terms), so compared on the scale of
            # the matching weight gradient
            w = n[: -len("bias")] + "weight"
            errs["d" + n] = max_abs(gb[n], ga[n]) / max(float(ga[w].abs().max()), 1e-30)
        else:
            errs["d" + n] = max_rel(gb[n], ga[n])
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:6]
    _say(f"[C3 fp32 B=2] loss {float(sa):.6f} vs {float(sb):.6f}; worst {worst}")
    bad = {n: e for n, e in errs.items() if e > 1e-4}
    assert not bad, bad


class _TorchPathAttention(DisentangledSelfAttention):
    """The module forced onto its torch-operation path (deberta_amd.unfused,
    held to the oracle module on the CPU in tests/test_module_cpu.py and
    tests/test_unfused_cpu.py): output_attentions on, the probabilities
    dropped."""

    def forward(self, hidden_states, attention_mask, output_attentions=False, query_states=None,
                relative_pos=None, rel_embeddings=None):
        ctx, _ = super().forward(hidden_states, attention_mask, True, query_states, relative_pos, rel_embeddings)
        return ctx, None


def test_c3_encoder_full_size_bf16(gpu):
    """C3 at its full size (B = 16, L = 512, bf16 autocast): forward and
    backward of the RTD loss with the fused attention in every layer against
    the same encoder (same fused blocks, weights, ids and labels) with the
    attention on its torch-operation path.  Both run bf16 under autocast, so
    they differ by bf16 rounding along 12 layers: the logits to 2e-2
    absolute, the loss to 1e-3, every parameter gradient to 3e-2 of its
    scale (a 12-layer chain of bf16 products; the single-layer bar of 2e-2
    holds for each layer in test_gpu_module.py)."""
    model = _encoder.Encoder(DisentangledSelfAttention, fused_blocks=True)
    _encoder.init_weights(model, seed=0)
    model = model.to(gpu)
    ids, labels = _encoder.synthetic_batch(16, 512, seed=0)
    mask = torch.ones(16, 1, 1, 512, dtype=torch.bool, device=gpu)
    rp = eager.relative_positions(512, 512, _encoder.BUCKETS, _encoder.MAX_POS).to(gpu)
    logits, loss, grads = _encoder_step(model, ids.to(gpu), labels.to(gpu), rp, mask, autocast=True)
    assert torch.isfinite(logits).all() and torch.isfinite(loss)
    assert abs(float(loss) - 0.693) < 0.2
    for n, g in grads.items():
        assert torch.isfinite(g).all(), n
    ref = _encoder.Encoder(_TorchPathAttention, fused_blocks=True).to(gpu)
    ref.load_state_dict(model.state_dict(), strict=True)
    del model
    torch.cuda.empty_cache()
    rlogits, rloss, rgrads = _encoder_step(ref, ids.to(gpu), labels.to(gpu), rp, mask, autocast=True)
    errs = {n: max_rel(grads[n], rgrads[n]) for n in grads if not n.endswith("self.key_proj.bias")}
    worst = sorted(errs.items(), key=lambda kv: -kv[1])[:6]
    labs, lossd = max_abs(logits, rlogits), abs(float(loss) - float(rloss))
    _say(f"[C3 bf16 B=16 vs torch path] loss {float(loss):.5f} vs {float(rloss):.5f}; logits max|err| {labs:.3e}; "
         f"worst grads {worst}")
    assert labs <= 2e-2 and lossd <= 1e-3
    bad = {n: e for n, e in errs.items() if e > 3e-2}
    assert not bad, bad
