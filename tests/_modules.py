"""Module-level helpers for the GPU parity tests: the oracle's restatement of
the reference module (CPU) and the fused module (GPU) with identical
weights, run on identical inputs, with gradients of the input, of the
relative-embedding table and of every parameter."""

from __future__ import annotations

import torch

from deberta_amd import DisentangledSelfAttention
from oracle import eager
from tests._cases import max_abs, max_rel


def _pair(cfg, seed=0):
    """Oracle module on the CPU and the fused module on the GPU with the
    same weights (N(0, 0.02), zero biases)."""
    torch.manual_seed(seed)
    ref = eager.EagerDisentangledSelfAttention(cfg)
    with torch.no_grad():
        for n, p in ref.named_parameters():
            p.copy_(torch.randn_like(p) * 0.02 if n.endswith("weight") else torch.zeros_like(p))
    ours = DisentangledSelfAttention(cfg)
    ours.load_state_dict(ref.state_dict(), strict=True)
    return ref.eval(), ours.eval()


def _run(module, x, mask, rel, device, autocast=False, relative_pos=None):
    x = x.to(device).detach().clone().requires_grad_(True)
    rel = rel.to(device).detach().clone().requires_grad_(True)
    m = mask.to(device) if mask is not None else None
    rp = relative_pos.to(device) if relative_pos is not None else None
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        out, _ = module(x, m, relative_pos=rp, rel_embeddings=rel)
    g = torch.Generator(device="cpu").manual_seed(123)
    dout = torch.randn(out.shape, generator=g).to(device=device, dtype=out.dtype)
    # a compiled module (torch.compile) names its parameters under _orig_mod.
    names = [n.removeprefix("_orig_mod.") for n, _ in module.named_parameters()]
    params = [p for _, p in module.named_parameters()]
    grads = torch.autograd.grad(out, [x, rel] + params, dout, allow_unused=True)
    res = {"out": out.detach().float().cpu(), "dx": grads[0].float().cpu(), "drel": grads[1].float().cpu()}
    for n, gr in zip(names, grads[2:]):
        res["d" + n] = torch.zeros(1) if gr is None else gr.float().cpu()
    return res


# Biases whose exact gradient is zero: adding a vector to every key (or to
# every row of the pos-key table) shifts each score row by a constant, which
# softmax ignores (sum_j dS_ij = 0).  They are compared on the scale of the
# matching weight gradient instead of their own (rounding-noise) scale.
_SHIFT_INVARIANT = {"dkey_proj.bias": "dkey_proj.weight", "dpos_key_proj.bias": "dpos_key_proj.weight"}


def _errors(ref: dict, got: dict) -> dict:
    errs = {}
    for k in ref:
        if k in _SHIFT_INVARIANT:
            scale = float(ref[_SHIFT_INVARIANT[k]].abs().max())
            errs[k] = max_abs(got[k], ref[k]) / max(scale, 1e-30)
        else:
            errs[k] = max_rel(got[k], ref[k])
    return errs
