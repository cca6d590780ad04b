"""GPU parity of the fused blocks around the attention (deberta_amd.blocks,
include/dsa_block.h) with the oracle's restatement of the reference blocks
(oracle/blocks.py), same weights and inputs, forward and every gradient
(input, residual, parameters).

Tolerances: fp32 max|err| / max|ref| <= 1e-4 per tensor.  bf16 (kernels fed
bf16, the oracle fp32 on the same rounded values): outputs and input
gradients |err| <= 2e-2 * max(1, |ref|) element by element (2e-2 absolute
for values up to 1, and relative above, since a LayerNorm output of size 8
held in bf16 is itself only exact to 3e-2); parameter gradients (sums over
every row) within 2e-2 of their scale.
"""

from __future__ import annotations

import sys

import pytest
import torch

from deberta_amd import FusedIntermediate, FusedOutput, FusedRTDHead, FusedSelfOutput, RelativeEmbeddings
from oracle import blocks as ob
from oracle import eager
from tests._cases import max_abs, max_rel

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _cfg():
    return eager.make_config(hidden_size=768, num_attention_heads=12, intermediate_size=3072, layer_norm_eps=1e-7,
                             norm_eps=1e-7, hidden_dropout_prob=0.0)


def _pair(ours_cls, ref_cls, seed, **kw):
    ref = ref_cls(_cfg(), **kw)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for n, p in ref.named_parameters():
            scale = 0.02 if p.dim() > 1 else 0.5
            p.copy_(torch.randn(p.shape, generator=g) * scale + (1.0 if n.endswith("LayerNorm.weight") or n == "norm.weight" else 0.0))
    ours = ours_cls(_cfg())
    ours.load_state_dict(ref.state_dict(), strict=True)
    return ref.eval(), ours.eval()


def _grads(module, inputs, run, device, dtype):
    xs = [t.to(device=device, dtype=dtype if t.is_floating_point() else t.dtype).detach().clone() for t in inputs]
    for t in xs:
        if t.is_floating_point():
            t.requires_grad_(True)
    out = run(module, *xs)
    g = torch.Generator().manual_seed(77)
    if out.dim() == 0:
        dout = torch.ones((), device=device)
    else:
        dout = torch.randn(out.shape, generator=g).to(device=device, dtype=out.dtype)
    leaves = [t for t in xs if t.requires_grad] + list(module.parameters())
    names = [f"d_in{i}" for i, t in enumerate(xs) if t.requires_grad] + ["d" + n for n, _ in module.named_parameters()]
    grads = torch.autograd.grad(out, leaves, dout, allow_unused=True)
    res = {"out": out.detach().float().cpu()}
    for n, gr in zip(names, grads):
        res[n] = torch.zeros(1) if gr is None else gr.detach().float().cpu()
    return res


def _compare(tag, ref, got, dtype, param_prefix="d", inputs_abs=("out", "d_in0", "d_in1")):
    errs = {}
    for k in ref:
        if dtype == torch.float32:
            errs[k] = max_rel(got[k], ref[k])
        elif k in inputs_abs:
            errs[k] = float(((got[k] - ref[k]).abs() / ref[k].abs().clamp(min=1.0)).max())
        else:
            errs[k] = max_rel(got[k], ref[k])
    _say(f"[{tag}] {errs}")
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    bad = {k: v for k, v in errs.items() if not v <= tol}
    assert not bad, bad


def _rnd(ts, dtype):
    return [t.to(dtype).float() if t.is_floating_point() else t for t in ts]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("kind", ["self", "ffn_out"])
def test_output_residual_norm(kind, dtype, gpu):
    """SelfOutput / Output: LayerNorm(dense(h) + input), 2 x 300 tokens
    (ragged row count), the dense GEMM plus the fused bias + residual +
    LayerNorm kernel."""
    if kind == "self":
        ref, ours = _pair(FusedSelfOutput, ob.OutputResidualNorm, 1)
        h_dim = 768
    else:
        ref, ours = _pair(FusedOutput, lambda c: ob.OutputResidualNorm(c, in_features=3072), 2)
        h_dim = 3072
    ours = ours.to(gpu, dtype)
    g = torch.Generator().manual_seed(3)
    h, inp = torch.randn(2, 300, h_dim, generator=g), torch.randn(2, 300, 768, generator=g)
    run = lambda m, a, b: m(a, b)
    want = _grads(ref if dtype == torch.float32 else _rounded(ref, dtype), _rnd([h, inp], dtype), run, "cpu", torch.float32)
    got = _grads(ours, [h, inp], run, gpu, dtype)
    _compare(f"{kind} {dtype}", want, got, dtype)


def _rounded(ref, dtype):
    """A copy of the oracle module with weights rounded to ``dtype`` (what
    the kernels read), kept in fp32."""
    import copy

    r = copy.deepcopy(ref)
    with torch.no_grad():
        for p in r.parameters():
            p.copy_(p.to(dtype).float())
    return r


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_intermediate(dtype, gpu):
    ref, ours = _pair(FusedIntermediate, ob.Intermediate, 4)
    ours = ours.to(gpu, dtype)
    h = torch.randn(2, 300, 768, generator=torch.Generator().manual_seed(5))
    run = lambda m, a: m(a)
    want = _grads(ref if dtype == torch.float32 else _rounded(ref, dtype), _rnd([h], dtype), run, "cpu", torch.float32)
    got = _grads(ours, [h], run, gpu, dtype)
    _compare(f"intermediate {dtype}", want, got, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("pairwise", [False, True])
def test_rtd_head_and_loss(dtype, pairwise, gpu):
    """RTDHead logits (CLS context, or none under a pairwise mask) and the
    fused classifier + BCE loss with inactive tokens, against the oracle
    head and discriminator loss."""
    ref, ours = _pair(FusedRTDHead, ob.RTDHead, 6)
    ours = ours.to(gpu, dtype)
    g = torch.Generator().manual_seed(7)
    h = torch.randn(2, 300, 768, generator=g)
    labels = (torch.rand(2, 300, generator=g) < 0.15).float()
    active = torch.rand(2, 300, generator=g) < 0.9
    mask = torch.ones(2, 1, 300, 300, dtype=torch.bool) if pairwise else None

    def run_ref(m, a):
        return ob.discriminator_loss(m(a, mask), labels, active)

    def run_ours(m, a):
        loss, logits = m.forward_loss(a, labels.to(gpu), active.to(gpu), None if mask is None else mask.to(gpu))
        plain = m(a, None if mask is None else mask.to(gpu))
        assert max_abs(plain.float().cpu(), logits.float().cpu()) <= (1e-4 if dtype == torch.float32 else 3e-2)
        return loss

    want = _grads(ref if dtype == torch.float32 else _rounded(ref, dtype), _rnd([h], dtype), run_ref, "cpu", torch.float32)
    got = _grads(ours, [h], run_ours, gpu, dtype)
    _compare(f"rtd pairwise={pairwise} {dtype}", want, got, dtype)


def test_relative_embeddings_layernorm(gpu):
    ref, ours = _pair(RelativeEmbeddings, ob.RelativeEmbeddings, 8)
    ours = ours.to(gpu)
    a, b = ref(), ours()
    assert max_rel(b.detach().cpu(), a.detach()) <= 1e-5
    ga = torch.autograd.grad(a, list(ref.parameters()), torch.ones_like(a))
    gb = torch.autograd.grad(b, list(ours.parameters()), torch.ones_like(b))
    for x, y in zip(ga, gb):
        assert max_rel(y.cpu(), x) <= 1e-4


def test_autocast_output_dtypes_follow_torch(gpu):
    """Under bf16 autocast the fused LayerNorm returns float32 (torch runs
    layer_norm in float32 there) and the fused GELU keeps the GEMM's bf16."""
    _, so = _pair(FusedSelfOutput, ob.OutputResidualNorm, 9)
    _, it = _pair(FusedIntermediate, ob.Intermediate, 10)
    so, it = so.to(gpu), it.to(gpu)
    x = torch.randn(4, 64, 768, device=gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = so(x, x)
        z = it(y)
        ref_y = torch.nn.functional.layer_norm(torch.nn.functional.linear(x, so.dense.weight, so.dense.bias) + x,
                                               (768,), so.LayerNorm.weight, so.LayerNorm.bias, 1e-7)
    assert y.dtype == ref_y.dtype == torch.float32 and z.dtype == torch.bfloat16
    assert max_abs(y, ref_y) <= 5e-2


def test_hidden_dropout_in_training(gpu):
    """Hidden dropout p > 0 in training: torch's dropout on the dense output
    (bias included), then the residual LayerNorm kernel.  With one seed the
    reference block in torch operations on the GPU draws the same mask, so
    the outputs and every gradient agree (fp32, 1e-4 of scale); the dropped
    share is near p."""
    cfg = _cfg()
    cfg.hidden_dropout_prob = 0.1
    ref = ob.OutputResidualNorm(cfg).to(gpu)
    ours = FusedSelfOutput(cfg).to(gpu)
    ours.load_state_dict(ref.state_dict(), strict=True)
    ref.train(), ours.train()
    g = torch.Generator().manual_seed(21)
    x = torch.randn(4, 128, 768, generator=g).to(gpu)
    res = torch.randn(4, 128, 768, generator=g).to(gpu)
    outs = []
    for m in (ref, ours):
        xs, rs = x.clone().requires_grad_(True), res.clone().requires_grad_(True)
        torch.manual_seed(5)
        out = m(xs, rs)
        dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(2)).to(gpu)
        grads = torch.autograd.grad(out, [xs, rs] + list(m.parameters()), dout)
        outs.append([out.detach()] + [gr.detach() for gr in grads])
    errs = [max_rel(b.cpu(), a.cpu()) for a, b in zip(*outs)]
    _say(f"[hidden dropout] {errs}")
    assert all(e <= 1e-4 for e in errs), errs
    with torch.no_grad():
        torch.manual_seed(6)
        kept = ours.dropout(torch.ones(1 << 20, device=gpu)).ne(0).float().mean()
    assert abs(float(kept) - 0.9) < 0.01


def test_gelu_matches_erf_over_a_dense_range(gpu):
    """The kernels' GELU takes erf from Abramowitz & Stegun 7.1.26 (|error
    of erf| <= 1.5e-7).  Over 2^20 fp32 values in [-12, 12], both the 8-wide
    kernels (C a multiple of 8) and the 4-wide ones (C = 12) against fp64
    gelu(z) = z Phi(z) and gelu'(z) = Phi(z) + z phi(z): forward within
    4e-7 * max(1, |z|), derivative within 1e-6."""
    from deberta_amd.blocks import _bias_gelu_bwd_impl, _bias_gelu_impl

    z64 = torch.linspace(-12.0, 12.0, 1 << 20, dtype=torch.float64)
    want = torch.nn.functional.gelu(z64)
    phi = torch.exp(-0.5 * z64 * z64) / (2.0 * torch.pi) ** 0.5
    want_d = 0.5 * (1.0 + torch.erf(z64 / 2.0 ** 0.5)) + z64 * phi
    for cols in (1024, 12):
        n = z64.numel() // cols
        z = z64[: n * cols].float().reshape(n, cols).to(gpu)
        y = _bias_gelu_impl(z, None).double().cpu().reshape(-1)
        dz, _ = _bias_gelu_bwd_impl(torch.ones_like(z), z, None)
        dz = dz.double().cpu().reshape(-1)
        zz = z64[: n * cols]
        err = ((y - want[: n * cols]).abs() / zz.abs().clamp(min=1.0)).max().item()
        err_d = (dz - want_d[: n * cols]).abs().max().item()
        _say(f"[gelu erf C={cols}] forward {err:.3e} derivative {err_d:.3e}")
        assert err <= 4e-7 and err_d <= 1e-6, (cols, err, err_d)
