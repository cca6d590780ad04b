"""The drop-in module on CPU tensors, and the relative_pos verdict cache.

The reference module is device-agnostic (deberta_v2_native.py:564-652) and
its own hot-path tests run on the CPU.  ``DisentangledSelfAttention`` (and
``disentangled_attention``, ``disentangled_attention_bias``) route CPU
tensors to the package's torch-operation path (``deberta_amd.unfused``);
these tests hold that route to the oracle's restatement of the reference
module with identical weights: output, probabilities and every gradient
(input, relative table, each parameter), fp32, max|err| / max|ref| <= 1e-5
per tensor (both sides fp32, differing in operation order only).

The cache tests alternate fresh Toeplitz and non-Toeplitz relative_pos
matrices of one shape (int32 and int64, so that the int64 copy the check
makes is a new temporary every call): every verdict must be the matrix's
own.
"""

from __future__ import annotations

import pytest
import torch

from deberta_amd import DisentangledSelfAttention, SegmentMask, disentangled_attention
from deberta_amd.attention import table_for
from deberta_amd.relpos import build_relative_position, table_from_matrix
from oracle import eager
from tests._cases import max_rel
from tests._modules import _errors

TOL = 1e-5


def _pair(cfg, seed=0):
    torch.manual_seed(seed)
    ref = eager.EagerDisentangledSelfAttention(cfg)
    with torch.no_grad():
        for n, p in ref.named_parameters():
            p.copy_(torch.randn_like(p) * 0.2 if n.endswith("weight") else torch.randn_like(p) * 0.1)
    ours = DisentangledSelfAttention(cfg)
    ours.load_state_dict(ref.state_dict(), strict=True)
    return ref.eval(), ours.eval()


def _cfg(types="c2p|p2c", share=False, relative=True):
    # buckets 8 / max_pos 16 at L=24: offsets beyond the log region, saturated rows
    return eager.make_config(
        hidden_size=64, num_attention_heads=4, position_buckets=8, max_relative_positions=16,
        pos_att_type=types, share_att_key=share, relative_attention=relative,
    )


def _mask(kind, B, L, g):
    if kind == "none":
        return None
    if kind == "padding":
        keep = torch.ones(B, L, dtype=torch.bool)
        keep[1, 17:] = False
        return keep[:, None, None, :]
    if kind == "int_padding":  # integer keep masks become != 0
        keep = torch.ones(B, L, dtype=torch.int64)
        keep[0, 9:] = 0
        return keep[:, None, None, :]
    if kind == "pair":
        keep = torch.rand(B, 1, L, L, generator=g) < 0.7
        keep[0, 0, 5, :] = False  # a dead query row keeping one edge
        keep[0, 0, 5, 0] = True
        return keep
    if kind == "segment":
        ids = torch.tensor([[1] * 10 + [2] * 9 + [0] * 5, [3] * 24])
        return SegmentMask(ids)
    raise ValueError(kind)


def _run(module, x, mask, rel, relative_pos=None, query_states=None, output_attentions=False):
    x = x.detach().clone().requires_grad_(True)
    rel = rel.detach().clone().requires_grad_(True)
    qs = None if query_states is None else query_states.detach().clone().requires_grad_(True)
    out, probs = module(
        x, mask, output_attentions=output_attentions, query_states=qs, relative_pos=relative_pos, rel_embeddings=rel
    )
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(123))
    params = list(module.named_parameters())
    leaves = [x, rel] + ([qs] if qs is not None else []) + [p for _, p in params]
    grads = torch.autograd.grad(out, leaves, dout, allow_unused=True)
    res = {"out": out.detach(), "dx": grads[0], "drel": torch.zeros(1) if grads[1] is None else grads[1]}
    rest = grads[2:]
    if qs is not None:
        res["dqs"], rest = rest[0], rest[1:]
    for (n, _), gr in zip(params, rest):
        res["d" + n] = torch.zeros(1) if gr is None else gr
    if output_attentions:
        res["probs"] = probs.detach()
    return res


@pytest.mark.parametrize("types", ["c2p|p2c", "c2p|p2c|p2p", "p2c", "c2p", "p2p"])
@pytest.mark.parametrize("share", [False, True])
@pytest.mark.parametrize("mask", ["none", "padding", "pair", "segment"])
def test_module_on_cpu_matches_oracle(types, share, mask):
    cfg = _cfg(types, share)
    ref, ours = _pair(cfg)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 24, 64, generator=g)
    rel = torch.randn(16, 64, generator=g)
    m = _mask(mask, 2, 24, g)
    m_ref = m.dense() if isinstance(m, SegmentMask) else m
    a = _run(ref, x, m_ref, rel)
    b = _run(ours, x, m, rel)
    errs = _errors(a, b)
    assert all(e <= TOL for e in errs.values()), errs


@pytest.mark.parametrize("rel_kind", ["canonical", "arbitrary", "rank4"])
def test_module_on_cpu_relative_pos_and_probs(rel_kind):
    """A given relative_pos (canonical, not a function of i - j, batch-shared
    rank 4), output_attentions and an integer mask on the CPU route."""
    ref, ours = _pair(_cfg("c2p|p2c|p2p"))
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 24, 64, generator=g)
    rel = torch.randn(16, 64, generator=g)
    rp = build_relative_position(24, 24, bucket_size=8, max_position=16)
    if rel_kind == "arbitrary":
        rp = torch.randint(-12, 13, (24, 24), generator=g)
    elif rel_kind == "rank4":
        rp = rp[None, None].expand(2, 1, 24, 24)
    m = _mask("int_padding", 2, 24, g)
    a = _run(ref, x, m, rel, relative_pos=rp, output_attentions=True)
    b = _run(ours, x, m, rel, relative_pos=rp, output_attentions=True)
    errs = _errors(a, b)
    assert all(e <= TOL for e in errs.values()), errs


def test_module_on_cpu_query_states_and_no_relative():
    ref, ours = _pair(_cfg("c2p|p2c"))
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 24, 64, generator=g)
    qs = torch.randn(2, 24, 64, generator=g)
    rel = torch.randn(16, 64, generator=g)
    errs = _errors(_run(ref, x, None, rel, query_states=qs), _run(ours, x, None, rel, query_states=qs))
    assert all(e <= TOL for e in errs.values()), errs
    # relative_attention off: plain scaled softmax attention
    ref, ours = _pair(_cfg("c2p|p2c", relative=False))
    errs = _errors(_run(ref, x, None, rel), _run(ours, x, None, rel))
    assert all(e <= TOL for e in errs.values()), errs


@pytest.mark.parametrize("types", ["c2p|p2c", "c2p|p2c|p2p", "p2c", "none"])
def test_bias_api_on_cpu_matches_oracle(types):
    tl = eager.pos_att_types(types if types != "none" else None)
    cfg = _cfg(types if types != "none" else "c2p")
    cfg.pos_att_type = types if types != "none" else None
    _, ours = _pair(cfg)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 4, 24, 16, generator=g)
    k = torch.randn(2, 4, 24, 16, generator=g)
    rel = torch.randn(16, 64, generator=g)
    sf = 1 + len(tl)
    with torch.no_grad():
        got = ours.disentangled_attention_bias(q, k, None, rel, sf)
        kr = ours.key_proj(rel).view(16, 4, 16).permute(1, 0, 2) if ours.pos_key_proj is None else None
        kr = ours.pos_key_proj(rel).view(16, 4, 16).permute(1, 0, 2) if ours.pos_key_proj is not None else kr
        qr = ours.pos_query_proj(rel).view(16, 4, 16).permute(1, 0, 2) if ours.pos_query_proj is not None else None
        want = eager.relative_bias(q, k, kr, qr, eager.relative_positions(24, 24, 8, 16), 8, tl, sf, 16)
    assert got.shape == (2, 4, 24, 24) and got.dtype == q.dtype
    assert max_rel(got, want) <= TOL


@pytest.mark.parametrize("layout", ["bhld", "blhd"])
def test_functional_on_cpu_matches_oracle(layout):
    g = torch.Generator().manual_seed(9)
    B, H, L, D, A = 2, 3, 24, 16, 8
    q, k, v = (torch.randn(B, H, L, D, generator=g) for _ in range(3))
    kr, qr = torch.randn(H, 2 * A, D, generator=g), torch.randn(H, 2 * A, D, generator=g)
    keep = torch.ones(B, L, dtype=torch.bool)
    keep[0, 20:] = False
    m = keep[:, None, None, :]
    rel = eager.relative_positions(L, L, A, 16)
    want, _ = eager.attend(q, k, v, kr, qr, rel, m, types=["c2p", "p2c"], att_span=A)
    args = (q, k, v) if layout == "bhld" else tuple(t.transpose(1, 2) for t in (q, k, v))
    got = disentangled_attention(
        *args, kr, qr, None, m, position_buckets=A, max_relative_positions=16, layout=layout,
    )
    if layout == "blhd":
        got = got.transpose(1, 2)
    assert max_rel(got, want) <= TOL


def _toeplitz(L, g, dtype):
    rp = build_relative_position(L, L, bucket_size=8, max_position=16)
    return rp.to(dtype).clone()


def _not_toeplitz(L, g, dtype):
    rp = build_relative_position(L, L, bucket_size=8, max_position=16)
    i, j = torch.randint(0, L, (2,), generator=g).tolist()
    rp[i, j] += 1 + int(torch.randint(0, 3, (1,), generator=g))
    return rp.to(dtype).clone()


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_toeplitz_verdict_is_the_matrix_own(dtype):
    """200 fresh matrices of one shape, alternating Toeplitz and not: the
    check's temporaries (the int64 copy, the slice) reuse the same freed
    blocks, so a verdict keyed by their address would be inherited.  Every
    non-Toeplitz matrix is refused and every Toeplitz one accepted with its
    own table."""
    g = torch.Generator().manual_seed(0)
    L = 24
    want = table_from_matrix(build_relative_position(L, L, bucket_size=8, max_position=16))
    for n in range(200):
        if n % 2 == 0:
            t = table_for(_toeplitz(L, g, dtype), L, L, 8, 16, "cpu")
            assert torch.equal(t, want), n
            assert table_for(_toeplitz(L, g, dtype), L, L, 8, 16, "cpu", strict=False) is not None
        else:
            with pytest.raises(ValueError, match="depend on i - j"):
                table_for(_not_toeplitz(L, g, dtype), L, L, 8, 16, "cpu")
            assert table_for(_not_toeplitz(L, g, dtype), L, L, 8, 16, "cpu", strict=False) is None


def test_toeplitz_verdict_follows_in_place_writes_and_inference_tensors():
    rp = build_relative_position(24, 24, bucket_size=8, max_position=16)
    assert table_for(rp, 24, 24, 8, 16, "cpu") is not None
    rp[3, 5] += 1  # the same object, a new version
    assert table_for(rp, 24, 24, 8, 16, "cpu", strict=False) is None
    rp[3, 5] -= 1
    assert table_for(rp, 24, 24, 8, 16, "cpu") is not None
    # the same object sliced to another extent is checked at that extent
    assert table_for(rp, 20, 20, 8, 16, "cpu") is not None
    with torch.inference_mode():  # no version counter: checked on every call
        good = build_relative_position(24, 24, bucket_size=8, max_position=16)
        bad = good.clone()
        bad[0, 7] = 99
        for _ in range(3):
            assert table_for(good, 24, 24, 8, 16, "cpu") is not None
            assert table_for(bad, 24, 24, 8, 16, "cpu", strict=False) is None


def test_module_on_cpu_alternating_relative_pos():
    """The module, called with fresh canonical and non-canonical int32
    matrices in turn, matches the oracle on every call."""
    ref, ours = _pair(_cfg("c2p|p2c"))
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 24, 64, generator=g)
    rel = torch.randn(16, 64, generator=g)
    with torch.no_grad():
        for n in range(8):
            rp = (_toeplitz if n % 2 == 0 else _not_toeplitz)(24, g, torch.int32)
            a, _ = ref(x, None, relative_pos=rp, rel_embeddings=rel)
            b, _ = ours(x, None, relative_pos=rp, rel_embeddings=rel)
            assert max_rel(b, a) <= TOL, n


@pytest.mark.parametrize("types", ["c2p", "p2c"])
def test_bias_api_on_cpu_casts_tables_to_query_dtype(types, monkeypatch):
    """The reference's dtype contract of the relative products
    (tests/test_smoke.py:1904-1965, :1968-2029) on the CPU route: bf16
    projected tables meet float32 layers in float32."""
    from tests._modules import bias_dtype_contract

    assert bias_dtype_contract(types, torch.device("cpu"), monkeypatch) <= TOL
