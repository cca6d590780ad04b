"""Module-level parity on the GPU: deberta_amd.DisentangledSelfAttention
(fused HIP kernels) against the oracle's restatement of the reference module
with identical weights, including the gradients of the projection weights
and of the relative-embedding table; the torch.compile path; and
full-size properties of the op at the headline shape.

Tolerances as in test_gpu_parity.py: fp32 max|err|/max|ref| <= 1e-4;
bf16 (autocast) max|err| <= 2e-2 against the fp32 oracle.
"""

from __future__ import annotations

import math
import sys

import pytest
import torch

from deberta_amd import DisentangledSelfAttention
from oracle import eager
from tests._cases import max_abs, max_rel
from tests._modules import _errors, _pair, _run

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _config1(share=False, **kw):
    return eager.make_config(
        hidden_size=128, num_attention_heads=4, position_buckets=256, max_relative_positions=512,
        share_att_key=share, **kw,
    )


@pytest.mark.parametrize("share", [False, True])
@pytest.mark.parametrize("mask", ["none", "padding"])
def test_config1_fp32(share, mask, gpu):
    """BASELINE config 1 (B=2, L=128, hidden 128, 4 heads x 32, buckets 256,
    max_rel 512, rel table [512, 128]), fp32, forward and backward."""
    cfg = _config1(share)
    ref, ours = _pair(cfg)
    ours = ours.to(gpu)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 128, 128, generator=g)
    rel = torch.randn(512, 128, generator=g) * 0.02
    m = None
    if mask == "padding":
        keep = torch.ones(2, 128, dtype=torch.bool)
        keep[1, 77:] = False
        m = keep[:, None, None, :]
    a = _run(ref, x, m, rel, "cpu")
    b = _run(ours, x, m, rel, gpu)
    errs = _errors(a, b)
    _say(f"[module fp32 share={share} mask={mask}] {errs}")
    assert all(e <= 1e-4 for e in errs.values()), errs


def test_bf16_autocast_base_shape(gpu):
    """config-2 layer shape (hidden 768, 12 heads x 64) on 2 rows of 512,
    under bf16 autocast, against the fp32 oracle: the output and the input
    gradient max|err| <= 2e-2 (the north star's bf16 bound), the relative
    table's and every parameter's gradient max|err| / max|ref| <= 2e-2."""
    cfg = eager.make_config(hidden_size=768, num_attention_heads=12, share_att_key=True)
    ref, ours = _pair(cfg, seed=1)
    ours = ours.to(gpu)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 512, 768, generator=g)
    rel = torch.randn(512, 768, generator=g)
    keep = torch.ones(2, 512, dtype=torch.bool)
    keep[1, 300:] = False
    m = keep[:, None, None, :]
    a = _run(ref, x, m, rel, "cpu")
    b = _run(ours, x, m, rel, gpu, autocast=True)
    # Under autocast the projections themselves run in bf16, and parameter
    # gradients sum over every row: those are compared relative to their
    # scale; the output and the input gradient absolutely.
    errs = _errors(a, b)
    abs_errs = {k: max_abs(b[k], a[k]) for k in ("out", "dx")}
    _say(f"[module bf16 autocast] abs {abs_errs} rel-to-scale {errs}")
    assert all(e <= 2e-2 for e in abs_errs.values()), abs_errs
    assert all(e <= 2e-2 for k, e in errs.items() if k not in abs_errs), errs


def test_explicit_relative_pos_matches_none(gpu):
    cfg = _config1()
    _, ours = _pair(cfg)
    ours = ours.to(gpu)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 128, 128, generator=g).to(gpu)
    rel = (torch.randn(512, 128, generator=g) * 0.02).to(gpu)
    from deberta_amd import build_relative_position

    rp = build_relative_position(128, 128, bucket_size=256, max_position=512, device=gpu)
    with torch.no_grad():
        a, _ = ours(x, None, rel_embeddings=rel)
        b, _ = ours(x, None, relative_pos=rp[None, None], rel_embeddings=rel)
    assert torch.equal(a, b)
    # a matrix that is not a function of i - j is used as given (the torch
    # path, whose parity is in test_gpu_unfused.py): only query row 3 moves
    bad = rp.clone()
    bad[3, 5] += 1
    with torch.no_grad():
        c, _ = ours(x, None, relative_pos=bad, rel_embeddings=rel)
    moved = (c - a).abs().amax(dim=(0, 2))
    assert float(moved[3]) > 0 and float(moved[torch.arange(128) != 3].max()) <= 1e-5


def test_none_mask_equals_all_ones_exactly(gpu):
    cfg = _config1()
    _, ours = _pair(cfg)
    ours = ours.to(gpu)
    x = torch.randn(2, 128, 128, device=gpu)
    rel = torch.randn(512, 128, device=gpu) * 0.02
    with torch.no_grad():
        a, _ = ours(x, None, rel_embeddings=rel)
        b, _ = ours(x, torch.ones(2, 1, 1, 128, dtype=torch.bool, device=gpu), rel_embeddings=rel)
        c, _ = ours(x, torch.ones(2, 1, 128, 128, dtype=torch.bool, device=gpu), rel_embeddings=rel)
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_torch_compile(backend, gpu):
    """The op traced by Dynamo through its fake implementation (config-5
    style, smaller): compiled forward + backward equal the eager op."""
    torch._dynamo.reset()
    cfg = eager.make_config(hidden_size=256, num_attention_heads=4, share_att_key=True)
    _, ours = _pair(cfg, seed=5)
    ours = ours.to(gpu).train()
    x = torch.randn(2, 256, 256, device=gpu)
    rel = torch.randn(512, 256, device=gpu)

    def loss_fn(mod, x, rel):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out, _ = mod(x, None, rel_embeddings=rel)
        return out.float().square().mean()

    compiled = torch.compile(ours, backend=backend, dynamic=False)
    le = loss_fn(ours, x, rel)
    ge = torch.autograd.grad(le, list(ours.parameters()))
    lc = loss_fn(compiled, x, rel)
    gc = torch.autograd.grad(lc, list(ours.parameters()))
    assert torch.isfinite(lc) and abs(float(lc) - float(le)) <= 1e-3 * abs(float(le)) + 1e-6
    for a, b in zip(ge, gc):
        assert torch.isfinite(b).all()
        assert max_abs(b, a) <= 2e-2 * max(1.0, float(a.abs().max()))


def test_full_headline_shape_batch_consistency(gpu):
    """At the headline shape (B=32, L=512, H=12, D=64, bf16) the op is
    computed per (batch, head) item: the forward and dq/dk/dv of the full
    batch equal those of each batch row run alone, bit for bit, and the
    relative-table gradients equal the sum over rows."""
    from deberta_amd.relpos import relative_offset_table

    B, L, H, D, A = 32, 512, 12, 64, 256
    g = torch.Generator().manual_seed(9)
    mk = lambda *s: torch.randn(*s, generator=g).to(gpu, torch.bfloat16)
    q, k, v, dO = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, 2 * A, D), mk(H, 2 * A, D)
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=gpu)
    scale = 1 / math.sqrt(D * 3)

    def run(sl):
        ls = [t[sl].detach().clone().requires_grad_(True) for t in (q, k, v)]
        lr = [t.detach().clone().requires_grad_(True) for t in (kr, qr)]
        out, lse, _, _ = torch.ops.deberta_amd.dsa_fwd(*ls, *lr, table, None, None, A, scale)
        gr = torch.autograd.grad(out, ls + lr, dO[sl])
        return out, lse, gr

    out, lse, gr = run(slice(None))
    assert torch.isfinite(out).all() and all(torch.isfinite(x).all() for x in gr)
    dkr_sum = torch.zeros_like(gr[3], dtype=torch.float32)
    for b in (0, 13, 31):
        o1, l1, g1 = run(slice(b, b + 1))
        assert torch.equal(o1, out[b : b + 1]) and torch.equal(l1, lse[b : b + 1])
        for x, y in zip(g1[:3], gr[:3]):
            assert torch.equal(x, y[b : b + 1])
    for b in range(B):
        dkr_sum += run(slice(b, b + 1))[2][3].float()
    assert max_rel(gr[3].float(), dkr_sum) <= 2e-2


@pytest.mark.parametrize("share", [True, False])
def test_query_states_against_oracle(share, gpu):
    """``query_states`` (deberta_v2_native.py:585-588: the query projection
    reads them instead of the hidden states) on the fused module: output and
    the gradients of the hidden states, the query states, the relative
    embeddings and every parameter against the oracle module, fp32, max|err|
    / max|ref| <= 1e-4 (key biases on their weights' scale)."""
    cfg = eager.make_config(hidden_size=128, num_attention_heads=4, share_att_key=share,
                            pos_att_type="c2p|p2c", position_buckets=256, max_relative_positions=512)
    ref, ours = _pair(cfg, seed=5)
    ours = ours.to(gpu)
    g = torch.Generator().manual_seed(66)
    x = torch.randn(2, 160, 128, generator=g)
    qs = torch.randn(2, 160, 128, generator=g)
    rel = torch.randn(512, 128, generator=g)
    dout = torch.randn(2, 160, 128, generator=g)

    def run(module, dev):
        xx, qq, rr = (t.to(dev).clone().requires_grad_(True) for t in (x, qs, rel))
        out, _ = module(xx, None, query_states=qq, rel_embeddings=rr)
        params = [p for _, p in module.named_parameters()]
        grads = torch.autograd.grad(out, [xx, qq, rr] + params, dout.to(dev), allow_unused=True)
        res = {"out": out.detach().float().cpu()}
        for n, gr in zip(["dx", "dqs", "drel"] + ["d" + n for n, _ in module.named_parameters()], grads):
            res[n] = torch.zeros(1) if gr is None else gr.float().cpu()
        return res

    a = run(ref, "cpu")
    b = run(ours, gpu)
    errs = _errors(a, b)
    _say(f"[query_states share={share}] {errs}")
    assert all(e <= 1e-4 for e in errs.values()), errs


def test_alternating_relative_pos_matches_oracle_every_call(gpu):
    """Fresh int32 relative_pos matrices of one shape, canonical and not in
    turn (the module's int64 copy of each is a new temporary that reuses
    freed blocks): every call matches the oracle with that call's matrix
    (canonical ones on the kernels, the others on the torch path)."""
    cfg = _config1()
    ref, ours = _pair(cfg)
    ours = ours.to(gpu)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 128, 128, generator=g)
    rel = torch.randn(512, 128, generator=g) * 0.02
    from deberta_amd import build_relative_position

    canon = build_relative_position(128, 128, bucket_size=256, max_position=512)
    errs = []
    with torch.no_grad():
        for n in range(12):
            rp = canon.clone()
            if n % 2:
                i, j = torch.randint(0, 128, (2,), generator=g).tolist()
                rp[i, j] += 3
            rp = rp.to(torch.int32)
            want, _ = ref(x, None, relative_pos=rp, rel_embeddings=rel)
            got, _ = ours(x.to(gpu), None, relative_pos=rp.to(gpu), rel_embeddings=rel.to(gpu))
            errs.append(max_rel(got.cpu(), want))
    _say(f"[alternating relative_pos] {errs}")
    assert all(e <= 1e-4 for e in errs), errs
