"""Pins of the attention oracle (oracle/eager.py) — CPU only.

The reference's tests hold no golden vectors for this path (only
invariants), so the eager restatement is pinned by:
  * an independent fp64 brute force written from the math (oracle/brute.py):
    forward and analytic gradients, with every mask form;
  * the textbook special case (no relative terms) against
    torch.nn.functional.scaled_dot_product_attention;
  * the reference's own invariant tests, restated: variant agreement
    (test_smoke.py:1806, 2178), scale ratios (:2072, :2126), mask invariants
    (:2267, :2301, :2335, :2422, :2455, :2504), the doc-block mask (:322);
  * fp64 gradcheck.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import brute, eager

F64 = torch.float64


def _case(B=2, H=2, L=12, D=8, A=8, seed=0, mask="none"):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, L, D, generator=g, dtype=F64) for _ in range(3))
    kr, qr = (torch.randn(H, 2 * A, D, generator=g, dtype=F64) for _ in range(2))
    dO = torch.randn(B, H, L, D, generator=g, dtype=F64)
    keep = None
    if mask == "key":
        keep = torch.rand(B, L, generator=g) < 0.7
        keep[:, 0] = True
        m4 = keep[:, None, None, :]
    elif mask in ("pair", "dead"):
        keep = torch.rand(B, L, L, generator=g) < 0.6
        live = torch.ones(B, L, dtype=torch.bool) if mask == "pair" else torch.rand(B, L, generator=g) < 0.6
        eye = torch.eye(L, dtype=torch.bool)
        keep = (keep & ~eye) | (eye & live[:, :, None])
        m4 = keep[:, None]
    else:
        m4 = None
    return q, k, v, kr, qr, dO, keep, m4


TYPES = [["c2p", "p2c"], ["c2p"], ["p2c"], []]


@pytest.mark.parametrize("types", TYPES, ids=lambda t: "|".join(t) or "none")
@pytest.mark.parametrize("mask", ["none", "key", "pair", "dead"])
@pytest.mark.parametrize("buckets,max_pos", [(8, 16), (-1, 16)])
def test_eager_matches_brute_force(types, mask, buckets, max_pos):
    A = buckets if buckets > 0 else max_pos
    q, k, v, kr, qr, dO, keep, m4 = _case(A=A, mask=mask, seed=len(types) * 7 + len(mask))
    L = q.shape[2]
    rel = eager.relative_positions(L, L, buckets, max_pos)
    use_rel = bool(types)
    kr_ = kr if "c2p" in types else None
    qr_ = qr if "p2c" in types else None
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, kr, qr)]
    out, probs = eager.attend(
        leaves[0], leaves[1], leaves[2],
        leaves[3] if kr_ is not None else None, leaves[4] if qr_ is not None else None,
        rel if use_rel else None, m4, types=types, att_span=A, use_relative=use_rel,
    )
    sf = 1 + len(types)
    scale = 1.0 / math.sqrt(q.shape[-1] * sf)
    O_b, P_b = brute.forward(
        q.numpy(), k.numpy(), v.numpy(),
        None if kr_ is None else kr.numpy(), None if qr_ is None else qr.numpy(),
        rel.numpy() if use_rel else None, None if keep is None else keep.numpy(),
        mask in ("pair", "dead"), scale, A,
    )
    assert torch.allclose(out, torch.from_numpy(O_b), atol=1e-12, rtol=1e-10)
    assert torch.allclose(probs, torch.from_numpy(P_b), atol=1e-12, rtol=1e-10)
    grads = torch.autograd.grad(out, leaves, dO, allow_unused=True)
    gb = brute.backward(
        dO.numpy(), q.numpy(), k.numpy(), v.numpy(),
        None if kr_ is None else kr.numpy(), None if qr_ is None else qr.numpy(),
        rel.numpy() if use_rel else None, None if keep is None else keep.numpy(),
        mask in ("pair", "dead"), scale, A,
    )
    for name, got in zip(("q", "k", "v", "kr", "qr"), grads):
        ref = gb[name]
        if ref is None:
            continue
        got = torch.zeros_like(torch.from_numpy(ref)) if got is None else got
        assert torch.allclose(got, torch.from_numpy(ref), atol=1e-11, rtol=1e-9), name


def test_brute_force_detects_a_swapped_index():
    """A p2c row taken as c(i-j) instead of p(i-j) must be caught."""
    q, k, v, kr, qr, dO, _, _ = _case(A=8)
    rel = eager.relative_positions(12, 12, 8, 16)
    good, _ = brute.forward(q.numpy(), k.numpy(), v.numpy(), None, qr.numpy(), rel.numpy(), None, False, 0.2, 8)
    bad, _ = brute.forward(q.numpy(), k.numpy(), v.numpy(), None, qr.numpy(), (-rel).numpy(), None, False, 0.2, 8)
    assert not torch.allclose(torch.from_numpy(good), torch.from_numpy(bad), atol=1e-6)


def test_no_relative_terms_is_sdpa():
    q, k, v, *_ = _case(L=16, D=8)
    for types in (["c2p", "p2c"], []):
        out, _ = eager.attend(q, k, v, None, None, None, None, types=types, att_span=8, use_relative=False)
        sf = 1 + len(types)
        ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=1.0 / math.sqrt(8 * sf))
        assert torch.allclose(out, ref, atol=1e-12)


def test_sdpa_with_key_padding():
    q, k, v, *_ = _case(L=10, D=8)
    keep = torch.ones(2, 10, dtype=torch.bool)
    keep[1, 6:] = False
    out, _ = eager.attend(q, k, v, None, None, None, keep[:, None, None, :], types=[], att_span=8, use_relative=False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q, k, v, attn_mask=keep[:, None, None, :], scale=1.0 / math.sqrt(8)
    )
    live = keep[:, None, :, None]
    assert torch.allclose(out, ref * live, atol=1e-12)
    assert float(out[1, :, 6:].abs().max()) == 0.0


@pytest.mark.parametrize("types", [["c2p", "p2c"], ["c2p", "p2c", "p2p"]])
def test_variants_agree(types):
    """test_smoke.py:1806 / :2178 restated: einsum and bmm bias variants agree."""
    q, k, v, kr, qr, *_ = _case(L=16, A=8)
    rel = eager.relative_positions(16, 16, 8, 16)
    a = eager.relative_bias(q, k, kr, qr, rel, 8, types, 1 + len(types), 8, "einsum")
    b = eager.relative_bias(q, k, kr, qr, rel, 8, types, 1 + len(types), 8, "bmm")
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


def test_scale_factor_ratio():
    """test_smoke.py:2126 restated: bias(sf=3) / bias(sf=12) = sqrt(12/3)."""
    q, k, v, kr, qr, *_ = _case(L=8, A=8)
    rel = eager.relative_positions(8, 8, -1, 8)
    s3 = eager.relative_bias(q, k, kr, qr, rel, 8, ["c2p", "p2c"], 3, 8)
    s12 = eager.relative_bias(q, k, kr, qr, rel, 8, ["c2p", "p2c"], 12, 8)
    assert float(s3.abs().mean() / s12.abs().mean()) == pytest.approx(2.0, rel=1e-9)


def test_p2p_only_bias_nonzero_and_scaled():
    """test_smoke.py:2032 / :2072 restated for the oracle's p2p term."""
    q, k, v, kr, qr, *_ = _case(L=8, A=8)
    rel = eager.relative_positions(8, 8, -1, 8)
    s2 = eager.relative_bias(q, k, kr, qr, rel, 8, ["p2p"], 2, 8)
    s8 = eager.relative_bias(q, k, kr, qr, rel, 8, ["p2p"], 8, 8)
    assert float(s2.abs().mean()) > 0
    assert float(s2.abs().mean() / s8.abs().mean()) == pytest.approx(2.0, rel=1e-9)


def _module(**kw):
    torch.manual_seed(0)
    cfg = eager.make_config(hidden_size=32, num_attention_heads=4, position_buckets=8, max_relative_positions=16, **kw)
    return eager.EagerDisentangledSelfAttention(cfg).double(), cfg


def test_none_mask_equals_all_ones_exactly():
    """test_smoke.py:2422 / :2504 restated."""
    m, cfg = _module()
    x = torch.randn(2, 8, 32, dtype=F64)
    rel_emb = torch.randn(16, 32, dtype=F64)
    a, _ = m(x, None, rel_embeddings=rel_emb)
    b, _ = m(x, torch.ones(2, 1, 1, 8, dtype=torch.bool), rel_embeddings=rel_emb)
    assert torch.equal(a, b)


def test_broadcast_mask_equals_dense_mask_exactly():
    """test_smoke.py:2455 restated."""
    m, cfg = _module()
    x = torch.randn(1, 8, 32, dtype=F64)
    rel_emb = torch.randn(16, 32, dtype=F64)
    keep = torch.tensor([[1, 1, 1, 1, 1, 0, 0, 0]], dtype=torch.bool)
    a, _ = m(x, keep[:, None, None, :], rel_embeddings=rel_emb)
    dense = (keep[:, :, None] & keep[:, None, :])[:, None]
    b, _ = m(x, dense, rel_embeddings=rel_emb)
    assert torch.equal(a, b)
    assert eager.encoder_mask(keep.long()).shape == (1, 1, 1, 8)


def test_pairwise_dead_row_is_zero():
    """test_smoke.py:2335 restated: a CLS fallback edge with a false diagonal
    leaves the row dead (zero output and probabilities)."""
    m, cfg = _module(relative_attention=False, pos_att_type="")
    x = torch.randn(1, 4, 32, dtype=F64)
    pair = torch.tensor([[[[1, 1, 0, 0], [1, 1, 0, 0], [0, 0, 1, 0], [1, 0, 0, 0]]]], dtype=torch.bool)
    out, probs = m(x, pair, output_attentions=True)
    assert torch.isfinite(out).all() and torch.isfinite(probs).all()
    assert float(out[0, 3].abs().max()) == 0.0
    assert float(probs[0, :, 3].abs().max()) == 0.0
    assert float(out[0, 0].abs().max()) > 0.0


@pytest.mark.parametrize("kind", ["all_masked", "random"])
def test_masked_outputs_finite(kind):
    """test_smoke.py:2267 / :2301 restated."""
    m, cfg = _module()
    x = torch.randn(2, 8, 32, dtype=F64)
    g = torch.Generator().manual_seed(7)
    keep = torch.zeros(2, 8, dtype=torch.bool) if kind == "all_masked" else torch.randint(0, 2, (2, 8), generator=g).bool()
    out, _ = m(x, keep[:, None, None, :], rel_embeddings=torch.randn(16, 32, dtype=F64))
    assert torch.isfinite(out).all()


def test_doc_block_mask_structure():
    """test_smoke.py:322 restated, for the oracle and the product."""
    from deberta_amd.masks import build_doc_block_mask

    doc_ids = torch.tensor([[1, 1, 1, 2, 2, 0]])
    for fn in (eager.doc_block_mask, build_doc_block_mask):
        m = fn(doc_ids)
        assert m.shape == (1, 6, 6) and m.dtype == torch.bool
        assert m[0, 0, 1] and m[0, 0, 2] and m[0, 3, 4]
        assert not m[0, 0, 3] and not m[0, 3, 0] and not m[0, 0, 5]
        assert all(bool(m[0, i, i]) for i in range(5)) and not m[0, 5, 5]
        assert m[0, 5, 0] and int(m[0, 5].sum()) == 1


def test_gradcheck_fp64():
    q, k, v, kr, qr, dO, keep, m4 = _case(B=1, H=1, L=6, D=4, A=4, mask="key")
    rel = eager.relative_positions(6, 6, 4, 8)

    def f(q, k, v, kr, qr):
        return eager.attend(q, k, v, kr, qr, rel, m4, types=["c2p", "p2c"], att_span=4)[0]

    inputs = tuple(t.clone().requires_grad_(True) for t in (q, k, v, kr, qr))
    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-5)


def test_keep_mask_contract():
    with pytest.raises(TypeError):
        eager.keep_mask([1, 0])
    with pytest.raises(ValueError):
        eager.keep_mask(torch.ones(2, 2))
    assert torch.equal(eager.keep_mask(torch.tensor([2, 0, -1])), torch.tensor([True, False, True]))


def test_encoder_mask_values_by_element():
    """The oracle's encoder mask (deberta_v2_native.py:1049-1068) element by
    element, from loops: rank 2 (B, S) -> (B, 1, 1, S) with value m[b, j];
    rank 3 (B, S, S) -> (B, 1, S, S) with m[b, i, j]; rank 4 with a head
    axis -> (B, 1, S, S) with OR over heads; integer masks are != 0.  The
    package's get_attention_mask gives the same tensors."""
    from deberta_amd.masks import get_attention_mask

    g = torch.Generator().manual_seed(0)
    B, H, S = 2, 3, 5
    m2 = torch.randint(0, 3, (B, S), generator=g)
    m3 = torch.rand(B, S, S, generator=g) < 0.5
    m4 = torch.rand(B, H, S, S, generator=g) < 0.3
    e2, e3, e4 = eager.encoder_mask(m2), eager.encoder_mask(m3), eager.encoder_mask(m4)
    assert e2.shape == (B, 1, 1, S) and e3.shape == (B, 1, S, S) and e4.shape == (B, 1, S, S)
    for b in range(B):
        for i in range(S):
            for j in range(S):
                assert bool(e2[b, 0, 0, j]) == (int(m2[b, j]) != 0)
                assert bool(e3[b, 0, i, j]) == bool(m3[b, i, j])
                assert bool(e4[b, 0, i, j]) == any(bool(m4[b, h, i, j]) for h in range(H))
    one_head = m4[:, :1]
    assert torch.equal(eager.encoder_mask(one_head), one_head)
    for m in (m2, m3, m4, one_head):
        assert torch.equal(get_attention_mask(m), eager.encoder_mask(m))
    with pytest.raises(ValueError, match="rank"):
        eager.encoder_mask(torch.ones(1, 1, 1, 1, 2, dtype=torch.bool))
    with pytest.raises(ValueError, match="rank"):
        get_attention_mask(torch.ones(1, 1, 1, 1, 2, dtype=torch.bool))


def test_canonical_rel_rank_handling_by_element():
    """The oracle's relative_pos normalisation (deberta_v2_native.py:235-271):
    None builds the canonical matrix; rank 4 takes [0, 0], rank 3 takes
    [0] (batch-shared only), rank 2 is used as is, all sliced to
    [:Lq, :Lk] and cast to long; other ranks raise.  Checked against
    matrices whose entries name their own indices, so a wrong pick of
    batch, head, row or column shows."""
    from deberta_amd.relpos import normalize_relative_pos

    def coded(*shape):
        return torch.arange(int(torch.tensor(shape).prod()), dtype=torch.int32).reshape(shape)

    Lq, Lk = 3, 4
    r4, r3, r2 = coded(2, 2, 5, 6), coded(2, 5, 6), coded(5, 6)
    want4 = torch.tensor([[r4[0, 0, i, j] for j in range(Lk)] for i in range(Lq)], dtype=torch.long)
    want3 = torch.tensor([[r3[0, i, j] for j in range(Lk)] for i in range(Lq)], dtype=torch.long)
    want2 = torch.tensor([[r2[i, j] for j in range(Lk)] for i in range(Lq)], dtype=torch.long)
    for given, want in ((r4, want4), (r3, want3), (r2, want2)):
        got = eager.canonical_rel(given, Lq, Lk, 8, 16)
        assert got.dtype == torch.long and torch.equal(got, want)
        assert torch.equal(normalize_relative_pos(given, Lq, Lk), want)
    assert torch.equal(eager.canonical_rel(None, Lq, Lk, 8, 16), eager.relative_positions(Lq, Lk, 8, 16))
    for bad in (torch.zeros(5, dtype=torch.long), torch.zeros(1, 1, 1, 3, 3, dtype=torch.long)):
        with pytest.raises(ValueError, match="rank"):
            eager.canonical_rel(bad, 3, 3, 8, 16)
        with pytest.raises(ValueError, match="rank"):
            normalize_relative_pos(bad, 3, 3)
