"""Pins of the oracle's module wrapper (oracle/eager.py,
EagerDisentangledSelfAttention) and of its p2p term — CPU only.

The module parity tests on the GPU compare the fused module with this
wrapper, so its parameter-to-head mapping (``heads``: the Linear output
viewed per head; ``project_rel``: the relative table projected per head,
deberta_v2_native.py:224-233, 273-296) and its output assembly
(``:646-650``) are pinned here against a formulation that shares none of
that code: per-head slices of the weight matrices ``W[h*D:(h+1)*D]`` in
explicit loops, the fp64 brute-force attention of oracle/brute.py, and the
output written back column block by column block.  A transposed operand,
a wrong head slice or a swapped projection fails these.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import brute, eager

F64 = torch.float64


def _module(share: bool, types: str, seed: int = 0, hidden: int = 16, heads: int = 2, buckets: int = 8, max_pos: int = 16):
    cfg = eager.make_config(
        hidden_size=hidden, num_attention_heads=heads, share_att_key=share, pos_att_type=types,
        position_buckets=buckets, max_relative_positions=max_pos, max_position_embeddings=max_pos,
    )
    torch.manual_seed(seed)
    m = eager.EagerDisentangledSelfAttention(cfg).double()
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn_like(p) * 0.3)  # nonzero biases: a misplaced bias shows
    return m.eval()


def _head_slice(linear: torch.nn.Linear, x: torch.Tensor, h: int, D: int) -> np.ndarray:
    """x @ W[hD:(h+1)D]^T + b[hD:(h+1)D], one row at a time."""
    W = linear.weight.detach().numpy()[h * D : (h + 1) * D]
    b = linear.bias.detach().numpy()[h * D : (h + 1) * D]
    xs = x.detach().numpy()
    out = np.zeros(xs.shape[:-1] + (D,))
    for idx in np.ndindex(*xs.shape[:-1]):
        out[idx] = W @ xs[idx] + b
    return out


@pytest.mark.parametrize("share", [False, True])
@pytest.mark.parametrize("use_query", [False, True])
def test_project_rel_is_per_head_slices(share, use_query):
    """Kr[h, r] = rel[r] @ W[hD:(h+1)D]^T + b[hD:(h+1)D], with W the
    key (query) projection when shared, else pos_key_proj (pos_query_proj)."""
    m = _module(share, "c2p|p2c")
    A, H, D = m.pos_ebd_size, m.num_attention_heads, m.attention_head_size
    rel = torch.randn(3 * A, 16, dtype=F64)  # longer than 2A: only the first 2A rows are used
    got = m.project_rel(rel, use_query=use_query).detach().numpy()
    if use_query:
        layer = m.query_proj if share else m.pos_query_proj
    else:
        layer = m.key_proj if share else m.pos_key_proj
    assert got.shape == (H, 2 * A, D)
    for h in range(H):
        np.testing.assert_allclose(got[h], _head_slice(layer, rel[: 2 * A], h, D), rtol=0, atol=1e-12)


def test_heads_is_per_head_slices():
    m = _module(False, "c2p|p2c")
    x = torch.randn(2, 5, 16, dtype=F64)
    got = m.heads(m.value_proj(x)).detach().numpy()  # (B, H, L, D)
    for h in range(m.num_attention_heads):
        np.testing.assert_allclose(got[:, h], _head_slice(m.value_proj, x, h, m.attention_head_size), rtol=0, atol=1e-12)


def _brute_module(m, x, rel_emb, keep, pairwise):
    """The module's forward from per-head slices and the brute-force
    attention: output column block h*D:(h+1)*D holds head h."""
    H, D, A = m.num_attention_heads, m.attention_head_size, m.pos_ebd_size
    types = m.pos_att_type
    B, L, _ = x.shape
    q = np.stack([_head_slice(m.query_proj, x, h, D) for h in range(H)], axis=1)
    k = np.stack([_head_slice(m.key_proj, x, h, D) for h in range(H)], axis=1)
    v = np.stack([_head_slice(m.value_proj, x, h, D) for h in range(H)], axis=1)
    kproj = m.key_proj if m.share_att_key else m.pos_key_proj
    qproj = m.query_proj if m.share_att_key else m.pos_query_proj
    need_k = "c2p" in types or "p2p" in types
    need_q = "p2c" in types or "p2p" in types
    kr = np.stack([_head_slice(kproj, rel_emb[: 2 * A], h, D) for h in range(H)]) if need_k else None
    qr = np.stack([_head_slice(qproj, rel_emb[: 2 * A], h, D) for h in range(H)]) if need_q else None
    rel = eager.relative_positions(L, L, m.position_buckets, m.max_relative_positions).numpy()
    sf = 1 + sum(t in types for t in ("c2p", "p2c", "p2p"))
    O, _ = brute.forward(
        q, k, v, kr, qr, rel, keep, pairwise, 1.0 / math.sqrt(D * sf), A,
        p2p="p2p" in types, c2p="c2p" in types, p2c="p2c" in types,
    )
    out = np.zeros((B, L, H * D))
    for h in range(H):
        out[:, :, h * D : (h + 1) * D] = O[:, h]
    return out


@pytest.mark.parametrize("share", [False, True])
@pytest.mark.parametrize("types", ["c2p|p2c", "c2p", "p2c", "p2p", "c2p|p2c|p2p"])
@pytest.mark.parametrize("mask", ["none", "key", "pair"])
def test_module_forward_matches_per_head_brute_force(share, types, mask):
    m = _module(share, types, seed=len(types) + 3 * share)
    B, L = 2, 11  # past mid = 4: log buckets in use
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, L, 16, generator=g, dtype=F64)
    rel_emb = torch.randn(2 * m.pos_ebd_size, 16, generator=g, dtype=F64)
    keep = m4 = None
    pairwise = mask == "pair"
    if mask == "key":
        keep = np.ones((B, L), dtype=bool)
        keep[1, 7:] = False
        m4 = torch.from_numpy(keep)[:, None, None, :]
    elif mask == "pair":
        keep = (torch.rand(B, L, L, generator=g) < 0.6).numpy() | np.eye(L, dtype=bool)[None]
        keep[0, 3, :] = False  # a dead row
        m4 = torch.from_numpy(keep)[:, None]
    with torch.no_grad():
        got, probs = m(x, m4, rel_embeddings=rel_emb)
    want = _brute_module(m, x, rel_emb, keep, pairwise)
    np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=1e-11)
    assert probs is None


def test_module_query_states_feed_the_queries_only():
    """query_states (deberta_v2_native.py:585-588) replace the hidden states
    in the query projection only."""
    m = _module(True, "c2p|p2c")
    g = torch.Generator().manual_seed(2)
    x = torch.randn(1, 6, 16, generator=g, dtype=F64)
    qs = torch.randn(1, 6, 16, generator=g, dtype=F64)
    rel_emb = torch.randn(16, 16, generator=g, dtype=F64)
    with torch.no_grad():
        a, _ = m(x, None, query_states=qs, rel_embeddings=rel_emb)
        b, _ = m(x, None, rel_embeddings=rel_emb)
    assert not torch.allclose(a, b)
    # rebuilt by hand: a module whose query projection maps x to the same
    # queries qs gives
    m2 = _module(True, "c2p|p2c")
    m2.load_state_dict(m.state_dict())
    sol = torch.linalg.lstsq(x[0], qs[0] @ m.query_proj.weight.T).solution  # x @ sol = qs @ Wq^T
    with torch.no_grad():
        m2.query_proj.weight.copy_(sol.T)
        # the relative query table must stay that of the original weights
        m2.share_att_key = False
        m2.pos_query_proj = m.query_proj
        m2.pos_key_proj = m.key_proj
        c, _ = m2(x, None, rel_embeddings=rel_emb)
    torch.testing.assert_close(a, c, rtol=0, atol=1e-9)


@pytest.mark.parametrize("types", [["p2p"], ["c2p", "p2p"], ["c2p", "p2c", "p2p"]])
def test_p2p_term_matches_brute_force_with_gradients(types):
    """oracle.attend's p2p term (deberta_v2_native.py:298-347: rows
    A + min(i, A - 1) of Qr against the c2p rows of Kr) forward and autograd
    against the brute force's analytic gradients, with L > A so that the
    row clamp is exercised."""
    A, L = 4, 11
    g = torch.Generator().manual_seed(5)
    B, H, D = 2, 2, 4
    q, k, v, dO = (torch.randn(B, H, L, D, generator=g, dtype=F64) for _ in range(4))
    kr, qr = (torch.randn(H, 2 * A, D, generator=g, dtype=F64) for _ in range(2))
    rel = eager.relative_positions(L, L, 2 * A, 2 * A)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, kr, qr)]
    ctx, _ = eager.attend(*leaves, rel, None, types=types, att_span=A)
    grads = torch.autograd.grad(ctx, leaves, dO, allow_unused=True)
    sf = 1 + len(types)
    s = 1.0 / math.sqrt(D * sf)
    np_ = lambda t: t.numpy()
    O, _ = brute.forward(np_(q), np_(k), np_(v), np_(kr), np_(qr), rel.numpy(), None, False, s, A,
                         p2p=True, c2p="c2p" in types, p2c="p2c" in types)
    np.testing.assert_allclose(ctx.detach().numpy(), O, rtol=0, atol=1e-12)
    bg = brute.backward(np_(dO), np_(q), np_(k), np_(v), np_(kr), np_(qr), rel.numpy(), None, False, s, A,
                        p2p=True, c2p="c2p" in types, p2c="p2c" in types)
    for name, got in zip(("q", "k", "v", "kr", "qr"), grads):
        got = np.zeros_like(bg[name]) if got is None else got.numpy()
        np.testing.assert_allclose(got, bg[name], rtol=0, atol=1e-11, err_msg=name)
