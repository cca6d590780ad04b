"""GPU tests of the module paths beside the plain fused call:

* ``output_attentions=True`` and a ``relative_pos`` that is not a function of
  ``i - j``: the module's torch-operation path (deberta_amd.unfused), against
  the oracle module (context, probabilities, input / table / parameter
  gradients);
* per-head ``(B, H, S, S)`` keep masks: the fused kernels with a
  head-strided pair mask, against the oracle;
* attention dropout in training mode.

Tolerances: fp32 max|err| / max|ref| <= 1e-4 per tensor; bf16 autocast
max|err| <= 2e-2 (outputs, probabilities) against the fp32 oracle, as in
test_gpu_module.py.
"""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import eager
from tests._cases import max_abs, max_rel
from tests._modules import _errors, _pair

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _cfg(**kw):
    return eager.make_config(hidden_size=128, num_attention_heads=4, position_buckets=32, max_relative_positions=64, **kw)


def _run(module, x, mask, rel, device, relative_pos=None, autocast=False):
    """Output, probabilities and gradients (input, table, parameters)."""
    x = x.to(device).detach().clone().requires_grad_(True)
    rel = rel.to(device).detach().clone().requires_grad_(True)
    m = mask.to(device) if mask is not None else None
    rp = relative_pos.to(device) if relative_pos is not None else None
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        out, probs = module(x, m, output_attentions=True, relative_pos=rp, rel_embeddings=rel)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(3)).to(device=device, dtype=out.dtype)
    names = [n for n, _ in module.named_parameters()]
    params = [p for _, p in module.named_parameters()]
    grads = torch.autograd.grad(out, [x, rel] + params, dout, allow_unused=True)
    res = {"out": out.detach().float().cpu(), "probs": probs.detach().float().cpu(),
           "dx": grads[0].float().cpu(), "drel": grads[1].float().cpu()}
    for n, gr in zip(names, grads[2:]):
        res["d" + n] = torch.zeros(1) if gr is None else gr.float().cpu()
    return res


def _inputs(L=96, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(2, L, 128, generator=g), torch.randn(64, 128, generator=g) * 0.02


@pytest.mark.parametrize("types", ["c2p|p2c", "c2p|p2c|p2p"])
@pytest.mark.parametrize("mask", ["none", "pair"])
def test_output_attentions_fp32(types, mask, gpu):
    ref, ours = _pair(_cfg(pos_att_type=types))
    ours = ours.to(gpu)
    x, rel = _inputs()
    m = None
    if mask == "pair":
        m = torch.rand(2, 1, 96, 96, generator=torch.Generator().manual_seed(1)) < 0.7
        m |= torch.eye(96, dtype=torch.bool)
        m[1, 0, 40, 40] = False  # dead query row
    a = _run(ref, x, m, rel, "cpu")
    b = _run(ours, x, m, rel, gpu)
    errs = _errors(a, b)
    _say(f"[output_attentions fp32 {types} {mask}] {errs}")
    assert all(e <= 1e-4 for e in errs.values()), errs


def test_output_attentions_bf16_autocast(gpu):
    ref, ours = _pair(_cfg())
    ours = ours.to(gpu)
    x, rel = _inputs()
    a = _run(ref, x, None, rel, "cpu")
    b = _run(ours, x, None, rel, gpu, autocast=True)
    errs = {k: max_abs(b[k], a[k]) for k in ("out", "probs")}
    _say(f"[output_attentions bf16] {errs}")
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_relative_pos_not_a_function_of_offset(gpu):
    """A relative_pos matrix with entries that do not depend on i - j alone
    is used as given (the reference's contract), through the torch path."""
    ref, ours = _pair(_cfg())
    ours = ours.to(gpu)
    x, rel = _inputs()
    rp = torch.randint(-40, 41, (96, 96), generator=torch.Generator().manual_seed(2))

    def run(module, device):
        xx = x.to(device).requires_grad_(True)
        rr = rel.to(device).requires_grad_(True)
        out, _ = module(xx, None, relative_pos=rp.to(device), rel_embeddings=rr)
        gx, gr = torch.autograd.grad(out, (xx, rr), torch.ones_like(out))
        return out.detach().cpu(), gx.cpu(), gr.cpu()

    a, b = run(ref, "cpu"), run(ours, gpu)
    errs = [max_rel(y, x_) for x_, y in zip(a, b)]
    _say(f"[non-Toeplitz relative_pos fp32] {errs}")
    assert all(e <= 1e-4 for e in errs), errs


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_per_head_pair_mask_on_the_kernels(dtype, gpu):
    """(B, H, S, S) keep masks run on the fused kernels (head-strided pair
    mask, per-head query liveness) and match the oracle, forward and
    backward, at a ragged length."""
    ref, ours = _pair(_cfg())
    ours = ours.to(gpu)
    L = 130
    x, rel = _inputs(L)
    g = torch.Generator().manual_seed(4)
    m = torch.rand(2, 4, L, L, generator=g) < 0.6
    m |= torch.eye(L, dtype=torch.bool)
    m[0, 1, 17, 17] = False  # a dead row in one head only
    m[1, 3, 100:, :] = False  # dead rows in another
    from tests._modules import _run as run_module

    a = run_module(ref, x, m, rel, "cpu")
    b = run_module(ours, x, m, rel, gpu, autocast=(dtype == "bf16"))
    if dtype == "fp32":
        errs = _errors(a, b)
        tol = 1e-4
    else:
        errs = {"out": max_abs(b["out"], a["out"])}
        tol = 2e-2
    _say(f"[per-head mask {dtype}] {errs}")
    assert all(e <= tol for e in errs.values()), errs


def test_attention_dropout_in_training(gpu):
    """Training with attention dropout p = 0.2: the returned probabilities
    are the eval-mode ones with about a fifth zeroed and the rest over 0.8,
    the context is those probabilities times the values, and the backward
    runs."""
    cfg = _cfg(attention_probs_dropout_prob=0.2)
    _, ours = _pair(cfg)
    ours = ours.to(gpu)
    x, rel = _inputs()
    xg, rg = x.to(gpu), rel.to(gpu)
    with torch.no_grad():
        _, plain = ours.eval()(xg, None, output_attentions=True, rel_embeddings=rg)
    ours.train()
    torch.manual_seed(0)
    xx = xg.clone().requires_grad_(True)
    out, probs = ours(xx, None, output_attentions=True, rel_embeddings=rg)
    kept = probs != 0
    frac = 1.0 - float(kept.float().mean())
    assert 0.17 < frac < 0.23, frac
    assert max_rel(probs[kept], plain[kept] / 0.8) <= 1e-5
    v = ours.value_proj(xg).view(2, 96, 4, 32).permute(0, 2, 1, 3)
    want = torch.matmul(probs, v).permute(0, 2, 1, 3).reshape(2, 96, 128)
    assert max_rel(out.detach(), want.detach()) <= 1e-5
    (gx,) = torch.autograd.grad(out, (xx,), torch.ones_like(out))
    assert torch.isfinite(gx).all()


def _plain_run(module, x, mask, rel, device, relative_pos=None):
    """Output and gradients without output_attentions (the module decides
    its path by itself)."""
    x = x.to(device).detach().clone().requires_grad_(True)
    rel = rel.to(device).detach().clone().requires_grad_(True)
    m = mask.to(device) if mask is not None else None
    rp = relative_pos.to(device) if relative_pos is not None else None
    out, _ = module(x, m, relative_pos=rp, rel_embeddings=rel)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(4)).to(device=device, dtype=out.dtype)
    names = [n for n, _ in module.named_parameters()]
    params = [p for _, p in module.named_parameters()]
    grads = torch.autograd.grad(out, [x, rel] + params, dout, allow_unused=True)
    res = {"out": out.detach().double().cpu(), "dx": grads[0].double().cpu(), "drel": grads[1].double().cpu()}
    for n, gr in zip(names, grads[2:]):
        res["d" + n] = torch.zeros(1) if gr is None else gr.double().cpu()
    return res


def test_head_dims_the_kernels_do_not_take_run_the_torch_path(gpu, monkeypatch):
    """The reference's own test shape (hidden 32, 4 heads, head dim 8) and
    head dim 128 on the GPU: the module runs the torch path (the kernels are
    switched off for the test) and matches the oracle module (fp32)."""
    import deberta_amd.attention as att

    def _no_kernels(*a, **k):
        raise AssertionError("the kernels ran")

    monkeypatch.setattr(att, "fused_attention", _no_kernels)
    for hidden, heads in ((32, 4), (256, 2)):
        cfg = eager.make_config(hidden_size=hidden, num_attention_heads=heads, position_buckets=32,
                                max_relative_positions=64)
        ref, ours = _pair(cfg)
        ours = ours.to(gpu)
        g = torch.Generator().manual_seed(hidden)
        x = torch.randn(2, 40, hidden, generator=g)
        rel = torch.randn(64, hidden, generator=g) * 0.02
        keep = torch.ones(2, 40, dtype=torch.bool)
        keep[1, 29:] = False
        m = keep[:, None, None, :]
        a = _plain_run(ref, x, m, rel, "cpu")
        b = _plain_run(ours, x, m, rel, gpu)
        errs = _errors(a, b)
        _say(f"[head dim {hidden // heads}] {errs}")
        assert all(e <= 1e-4 for e in errs.values()), errs


def test_float16_runs_the_torch_path(gpu, monkeypatch):
    """A float16 module on the GPU (the kernels take float32 and bfloat16):
    the torch path, against the oracle in float32 on the float16-rounded
    weights and inputs; output and input gradient to 2e-2 absolute."""
    import deberta_amd.attention as att

    def _no_kernels(*a, **k):
        raise AssertionError("the kernels ran")

    monkeypatch.setattr(att, "fused_attention", _no_kernels)
    ref, ours = _pair(_cfg())
    with torch.no_grad():
        for p_ in ref.parameters():
            p_.copy_(p_.half().float())
    ours.load_state_dict(ref.state_dict())
    ours = ours.to(gpu).half()
    x, rel = _inputs(seed=5)
    x, rel = x.half().float(), rel.half().float()
    a = _plain_run(ref, x, None, rel, "cpu")
    b = _plain_run(ours, x.half(), None, rel.half(), gpu)
    errs = {k: max_abs(b[k], a[k]) for k in ("out", "dx")}
    _say(f"[float16 module] {errs}")
    assert all(e <= 2e-2 for e in errs.values()), errs


def test_bias_api_with_a_matrix_used_as_given(gpu):
    """disentangled_attention_bias with a relative_pos that is not a function
    of i - j (the reference uses it as given) on the GPU equals the oracle's
    relative term (fp32, 1e-5 of scale)."""
    cfg = _cfg(pos_att_type="c2p|p2c")
    ref, ours = _pair(cfg)
    ours = ours.to(gpu)
    g = torch.Generator().manual_seed(6)
    B, H, L, D = 2, 4, 48, 32
    q, k = (torch.randn(B, H, L, D, generator=g) for _ in range(2))
    rel = torch.randn(64, 128, generator=g) * 0.02
    rp = eager.relative_positions(L, L, 32, 64).clone()
    rp[5, 7] += 3  # no longer Toeplitz
    got = ours.disentangled_attention_bias(q.to(gpu), k.to(gpu), rp.to(gpu), rel.to(gpu), 3)
    kr = ref.project_rel(rel, use_query=False)
    qr = ref.project_rel(rel, use_query=True)
    want = eager.relative_bias(q, k, kr, qr, eager.canonical_rel(rp, L, L, 32, 64), 32, ["c2p", "p2c"], 3, D, "einsum")
    err = max_rel(got.float().cpu(), want)
    _say(f"[bias api, matrix as given] {err:.2e}")
    assert err <= 1e-5
