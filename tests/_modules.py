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


def bias_dtype_contract(types: str, dev, monkeypatch) -> float:
    """The reference's dtype contract of the relative products
    (tests/test_smoke.py:1904-1965 and :1968-2029): projected tables that
    come back in bfloat16 (``_project_rel`` replaced) meet float32 query and
    key layers in float32 (head dim 32, the kernels' smallest, in place of
    the reference's 8).  Asserts a float32 bias of the right shape and
    returns its max|err| / max|ref| against the oracle's bias on the bf16
    tables widened to float32."""
    cfg = eager.make_config(hidden_size=128, num_attention_heads=4, max_position_embeddings=32,
                            position_buckets=-1, max_relative_positions=-1, pos_att_type=types)
    attn = DisentangledSelfAttention(cfg).to(dev).eval()
    A, H, D = int(attn.pos_ebd_size), 4, 32
    g = torch.Generator().manual_seed(19)
    tables = {u: torch.randn(H, 2 * A, D, generator=g).to(torch.bfloat16) for u in (False, True)}
    calls = []

    def fake_project_rel(rel, *, use_query):
        calls.append(use_query)
        return tables[use_query].to(dev)

    monkeypatch.setattr(attn, "_project_rel", fake_project_rel)
    B, L = 2, 40
    q = torch.randn(B, H, L, D, generator=g)
    k = torch.randn(B, H, L, D, generator=g)
    rel = torch.randn(2 * A, 128, generator=g)
    with torch.no_grad():
        got = attn.disentangled_attention_bias(q.to(dev), k.to(dev), None, rel.to(dev), 2)
    assert calls and got.dtype == torch.float32 and tuple(got.shape) == (B, H, L, L)
    kr = tables[False].float() if types == "c2p" else None
    qr = tables[True].float() if types == "p2c" else None
    want = eager.relative_bias(q, k, kr, qr, eager.relative_positions(L, L, -1, -1), A, [types], 2, D)
    return max_rel(got.float().cpu(), want)
