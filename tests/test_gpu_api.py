"""GPU tests of the rest of the reference's call surface on the fused
kernels: the bias API (``disentangled_attention_bias``,
deberta_v2_native.py:530-562) through ``dsa_bias``, the p2p term
(``:298-347``) carried by the c2p term's query rows, and the device-side
relative-position table at the bucket function's saturation edge.

Tolerances: fp32 max|err| / max|ref| <= 1e-4 (the north_star's "max
relative error" read relative to the tensor's scale, so that entries near
zero do not dominate); bf16 max|err| <= 2e-2 against the fp32 oracle on the
same bf16-rounded inputs.
"""

from __future__ import annotations

import math
import sys

import pytest
import torch

from deberta_amd import DisentangledSelfAttention, disentangled_attention
from deberta_amd.relpos import relative_offset_table
from oracle import eager
from tests._cases import max_abs, max_rel
from tests._modules import _errors, _pair, _run

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _bias_inputs(B, H, L, D, hidden, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, L, D, generator=g)
    k = torch.randn(B, H, L, D, generator=g)
    rel = torch.randn(512, hidden, generator=g)
    return q, k, rel


def _oracle_bias(ref, q, k, rel, types, sf, relative_pos=None):
    A = ref.pos_ebd_size
    kr = ref.project_rel(rel, use_query=False) if ("c2p" in types or "p2p" in types) else None
    qr = ref.project_rel(rel, use_query=True) if ("p2c" in types or "p2p" in types) else None
    rp = eager.canonical_rel(relative_pos, q.shape[2], k.shape[2], ref.position_buckets, ref.max_relative_positions)
    return eager.relative_bias(q, k, kr, qr, rp, A, types, sf, ref.attention_head_size)


@pytest.mark.parametrize("types", ["c2p|p2c", "c2p", "p2c", "p2p", "c2p|p2c|p2p"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("share", [False, True])
@pytest.mark.parametrize("D", [32, 64])
def test_bias_api_matches_oracle(types, dtype, share, D, gpu):
    """disentangled_attention_bias on the GPU against the oracle's bias
    (einsum + gather) at L = 300 (ragged tiles, log buckets in use), head
    dims 32 and 64 (hidden 128 over 4 or 2 heads)."""
    H = 128 // D
    cfg = eager.make_config(hidden_size=128, num_attention_heads=H, share_att_key=share, pos_att_type=types)
    ref, ours = _pair(cfg, seed=11)
    ours = ours.to(gpu)
    B, L = 2, 300
    q, k, rel = _bias_inputs(B, H, L, D, 128, seed=4)
    rnd = lambda t: t.to(dtype).float()
    types_l = eager.pos_att_types(types)
    sf = 1 + len(types_l)
    with torch.no_grad():
        want = _oracle_bias(ref, rnd(q), rnd(k), rel, types_l, sf)
        if dtype == torch.bfloat16:  # the tables the kernel reads are rounded too
            kr = ref.project_rel(rel, use_query=False).to(dtype).float() if ("c2p" in types_l or "p2p" in types_l) else None
            qr = ref.project_rel(rel, use_query=True).to(dtype).float() if ("p2c" in types_l or "p2p" in types_l) else None
            rp = eager.relative_positions(L, L, 256, 512)
            want = eager.relative_bias(rnd(q), rnd(k), kr, qr, rp, 256, types_l, sf, D)
        got = ours.disentangled_attention_bias(q.to(gpu, dtype), k.to(gpu, dtype), None, rel.to(gpu), sf)
    assert got.shape == (B, H, L, L) and got.dtype == dtype
    got = got.float().cpu()
    if dtype == torch.float32:
        err = max_rel(got, want)
        _say(f"[bias {types} fp32 D={D} share={share}] rel {err:.2e}")
        assert err <= 1e-4
    else:
        err = max_abs(got, want)
        _say(f"[bias {types} bf16 D={D} share={share}] abs {err:.2e} (max |ref| {float(want.abs().max()):.2f})")
        assert err <= 2e-2


def test_bias_api_recomputes_and_respects_scale_factor(gpu):
    """The reference's assertions on the bias API, restated at head dim 32
    (the kernels' smallest): tests/test_smoke.py:1853-1900 (a new query/key
    pair gives a new bias: nothing is cached across calls), :2072-2123 (p2p
    alone is nonzero and scales as sqrt(8 / 2)) and :2126-2175 (c2p|p2c
    scales as sqrt(12 / 3))."""
    cfg = eager.make_config(hidden_size=128, num_attention_heads=4, max_position_embeddings=32,
                            position_buckets=-1, max_relative_positions=-1, pos_att_type="c2p|p2c")
    attn = DisentangledSelfAttention(cfg).to(gpu).eval()
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(gpu)
    qa, ka, qb, kb = mk(2, 4, 8, 32), mk(2, 4, 8, 32), mk(2, 4, 8, 32), mk(2, 4, 8, 32)
    rel = mk(64, 128)
    with torch.no_grad():
        sa = attn.disentangled_attention_bias(query_layer=qa, key_layer=ka, relative_pos=None, rel_embeddings=rel, scale_factor=3)
        sb = attn.disentangled_attention_bias(query_layer=qb, key_layer=kb, relative_pos=None, rel_embeddings=rel, scale_factor=3)
        s12 = attn.disentangled_attention_bias(query_layer=qa, key_layer=ka, relative_pos=None, rel_embeddings=rel, scale_factor=12)
    assert sa.shape == sb.shape == (2, 4, 8, 8)
    assert not torch.allclose(sa, sb, rtol=0.0, atol=0.0) and float((sa - sb).abs().max()) > 0.0
    ratio = float(sa.abs().mean()) / float(s12.abs().mean())
    assert ratio == pytest.approx(math.sqrt(12.0 / 3.0), rel=1e-4, abs=1e-4)

    cfg_p = eager.make_config(hidden_size=128, num_attention_heads=4, max_position_embeddings=32,
                              position_buckets=-1, max_relative_positions=-1, pos_att_type="p2p")
    attn_p = DisentangledSelfAttention(cfg_p).to(gpu).eval()
    with torch.no_grad():
        p2 = attn_p.disentangled_attention_bias(query_layer=qa, key_layer=ka, relative_pos=None, rel_embeddings=rel, scale_factor=2)
        p8 = attn_p.disentangled_attention_bias(query_layer=qa, key_layer=ka, relative_pos=None, rel_embeddings=rel, scale_factor=8)
    assert torch.isfinite(p2).all() and float(p2.abs().sum()) > 0.0
    assert float(p2.abs().mean()) / float(p8.abs().mean()) == pytest.approx(math.sqrt(8.0 / 2.0), rel=1e-4, abs=1e-4)


def _p2p_config(share, types="c2p|p2c|p2p"):
    return eager.make_config(hidden_size=128, num_attention_heads=4, position_buckets=256, max_relative_positions=512,
                             share_att_key=share, pos_att_type=types)


@pytest.mark.parametrize("types", ["c2p|p2c|p2p", "p2p", "c2p|p2p", "p2c|p2p"])
@pytest.mark.parametrize("share", [False, True])
@pytest.mark.parametrize("mask", ["none", "padding"])
def test_p2p_module_parity_fp32(types, share, mask, gpu):
    """The module with the p2p term (deberta_v2_native.py:298-347) against the
    oracle module, fp32, forward and every gradient.  The p2p query rows
    A + min(i, A - 1) stop moving past i = A - 1 = 255, which L = 300
    exercises."""
    cfg = _p2p_config(share, types)
    ref, ours = _pair(cfg, seed=3)
    ours = ours.to(gpu)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 300, 128, generator=g)
    rel = torch.randn(512, 128, generator=g) * 0.5
    m = None
    if mask == "padding":
        keep = torch.ones(2, 300, dtype=torch.bool)
        keep[1, 211:] = False
        m = keep[:, None, None, :]
    a = _run(ref, x, m, rel, "cpu")
    b = _run(ours, x, m, rel, gpu)
    errs = _errors(a, b)
    _say(f"[p2p module fp32 {types} share={share} mask={mask}] {errs}")
    assert all(e <= 1e-4 for e in errs.values()), errs


def test_p2p_op_bf16(gpu):
    """The functional op with p2p in bf16 against the fp32 oracle on the
    same bf16-rounded inputs: max abs error <= 2e-2 on the output and on
    every gradient (q, k, v and both tables)."""
    B, H, L, D, A = 2, 4, 300, 64, 256
    g = torch.Generator().manual_seed(21)
    q, k, v, dO = (torch.randn(B, H, L, D, generator=g) for _ in range(4))
    kr, qr = (torch.randn(H, 2 * A, D, generator=g) for _ in range(2))
    bf = lambda t: t.to(torch.bfloat16)
    types = ["c2p", "p2c", "p2p"]
    lc = [bf(t).float().requires_grad_(True) for t in (q, k, v, kr, qr)]
    rel = eager.relative_positions(L, L, 256, 512)
    ctx, _ = eager.attend(*lc, rel, None, types=types, att_span=A)
    gc = torch.autograd.grad(ctx, lc, bf(dO).float())
    ld = [bf(t).to(gpu).requires_grad_(True) for t in (q, k, v, kr, qr)]
    out = disentangled_attention(*ld, None, None, position_buckets=256, max_relative_positions=512,
                                 att_type="c2p|p2c|p2p")
    gd = torch.autograd.grad(out, ld, bf(dO).to(gpu))
    errs = {"out": max_abs(out.detach().float().cpu(), ctx.detach())}
    for n, a_, b_ in zip(("dq", "dk", "dv", "dkr", "dqr"), gd, gc):
        errs[n] = max_abs(a_.float().cpu(), b_)
    _say(f"[p2p op bf16] {errs}")
    assert all(e <= 2e-2 for e in errs.values()), errs


@pytest.mark.parametrize("buckets,max_pos", [(256, 512), (128, 512)])
def test_device_bucket_table_matches_oracle(buckets, max_pos, gpu):
    """The relative-position table built on the GPU (the kernels' input)
    equals the CPU oracle's bucket function over |i - j| <= 4095, the
    saturation edge included: the device's fp32 log / ceil land on the same
    integers as the CPU's for every offset of a 4096-token sequence."""
    L = 4096
    dev = relative_offset_table(L, L, bucket_size=buckets, max_position=max_pos, device=gpu).cpu().long()
    d = torch.arange(-(L - 1), L)
    want = eager.log_bucket(d, buckets, max_pos)
    mid = buckets // 2
    edge = {int(x): int(dev[x + L - 1]) for x in (mid - 1, mid, max_pos - 2, max_pos - 1, max_pos, L - 1)}
    _say(f"[bucket table {buckets}/{max_pos}] values at the edges {edge}")
    assert torch.equal(dev, want)
    assert edge[L - 1] == edge[max_pos - 1] == -int(dev[0])  # saturated, odd


@pytest.mark.parametrize(
    "split",
    [
        ("PREP", "DKDV", "DQ|TABLE", "SUM"),
        ("PREP", "DKDV", "DQ", "TABLE", "SUM"),
        ("PREP", "DKDV", "DQ", "FOLD"),
        ("PREP", "DKDV", "DQ|FOLD"),
    ],
    ids=["dqtable-sum", "dq-table-sum", "dq-fold", "dqfold"],
)
def test_backward_stages_in_separate_calls(split, gpu):
    """dsa_bwd run as separate stage calls (include/dsa.h: PREP, DKDV, DQ,
    FOLD = TABLE then SUM) gives the one-call backward's results: dq, dk, dv
    bitwise; dkr, dqr up to the order of their fp32 atomic additions."""
    import ctypes

    from deberta_amd import _lib, ops

    lib = _lib.load()
    B, L, H, D, A = 2, 256, 4, 64, 256
    g = torch.Generator().manual_seed(31)
    mk = lambda *s: torch.randn(*s, generator=g).to(gpu, torch.bfloat16)
    q, k, v, dout = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, 2 * A, D), mk(H, 2 * A, D)
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=gpu)
    scale = 1 / math.sqrt(D * 3)
    out, lse, bias, _ = torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, A, scale)
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    bits = {"PREP": _lib.DSA_STAGE_PREP, "DQ": _lib.DSA_STAGE_DQ, "DKDV": _lib.DSA_STAGE_DKDV,
            "FOLD": _lib.DSA_STAGE_FOLD, "TABLE": _lib.DSA_STAGE_TABLE, "SUM": _lib.DSA_STAGE_SUM}

    def run(calls):
        grads = [torch.full_like(q, float("nan")) for _ in range(3)]
        tabs = [torch.zeros((H, 2 * A, D), dtype=torch.float32, device=gpu) for _ in range(2)]
        a = ops.fill_bwd_args(dout, q, k, v, kr, qr, table, None, None, out, lse, bias, A, scale, *grads, *tabs)
        ws = torch.empty((ops.bwd_workspace_bytes(a),), dtype=torch.uint8, device=gpu)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        for c in calls:
            a.stages = 0
            for s in c.split("|") if c else []:
                a.stages |= bits[s]
            _lib.check(lib.dsa_bwd(ctypes.byref(a), stream), "dsa_bwd")
        torch.cuda.synchronize(gpu)
        return grads + tabs

    _say(f"[stages] split {'/'.join(split)}")
    ref = run([""])
    got = run(list(split))
    for name, a, b in zip(["dq", "dk", "dv", "dkr", "dqr"], got, ref):
        if name in ("dkr", "dqr"):
            err = float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
            assert err <= 1e-5, f"{name} differs from the one-call backward ({err:.3e})"
        else:
            assert torch.equal(a, b), f"{name} differs from the one-call backward"


def _host_order_costs(seg, ntiles, per):
    """Launch-order costs from the segment ids on the host: 1 + the number of
    the other side's tiles (``per`` 32-token chunks each) whose segment range
    meets the 128-token tile's (ranges over nonzero ids; an empty range
    meets nothing), capped at 1025."""
    B, L = seg.shape
    nch = (L + 31) // 32
    pad = torch.zeros(B, nch * 32, dtype=torch.int64)
    pad[:, :L] = seg.long()
    big = 1 << 40
    lo = torch.where(pad > 0, pad, torch.full_like(pad, big)).view(B, nch, 32).amin(-1)
    hi = torch.where(pad > 0, pad, torch.full_like(pad, -big)).view(B, nch, 32).amax(-1)

    def ranges(width, n):
        out_lo = torch.full((B, n), big, dtype=torch.int64)
        out_hi = torch.full((B, n), -big, dtype=torch.int64)
        for t in range(n):
            c0, c1 = width * t, min(width * t + width, nch)
            if c0 < c1:
                out_lo[:, t] = lo[:, c0:c1].amin(-1)
                out_hi[:, t] = hi[:, c0:c1].amax(-1)
        return out_lo, out_hi

    mlo, mhi = ranges(4, ntiles)
    olo, ohi = ranges(per, (nch + per - 1) // per)
    meets = (
        (mlo[:, :, None] <= mhi[:, :, None]) & (olo[:, None, :] <= ohi[:, None, :])
        & (mlo[:, :, None] <= ohi[:, None, :]) & (olo[:, None, :] <= mhi[:, :, None])
    )
    return (1 + meets.sum(-1)).clamp_max(1025)


@pytest.mark.parametrize("B,L", [(4, 4096), (24, 2048)], ids=["C4", "B24"])
def test_forward_launch_order(B, L, gpu):
    """The forward's heaviest-first launch order under segment masks
    (dsa_order.h): the cost of every (batch row, 128-query tile) equals the
    host count, and the order is a permutation of the items with
    non-increasing cost."""
    import ctypes

    from deberta_amd import _lib, ops

    lib = _lib.load()
    H, D, A = 1, 64, 256
    g = torch.Generator().manual_seed(41)
    seg = torch.zeros(B, L, dtype=torch.int32)
    for b in range(B):  # packed documents with padding at the end of the row
        t, doc = 0, 1
        end = L - int(torch.randint(0, L // 4, (1,), generator=g))
        while t < end:
            n = min(int(torch.randint(1, 1200, (1,), generator=g)), end - t)
            seg[b, t:t + n] = doc
            t, doc = t + n, doc + 1
    mk = lambda *s: torch.randn(*s, generator=g).to(gpu, torch.bfloat16)
    q, k, v = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, 2 * A, D), mk(H, 2 * A, D)
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=gpu)
    segd = seg.to(gpu)
    out = torch.empty_like(q)
    lse = torch.empty((B, H, L), dtype=torch.float32, device=gpu)
    bias = torch.empty(ops.bias_shape(q, k), dtype=torch.float16, device=gpu)
    a = ops._fill_fwd_args(q, k, v, kr, qr, table, segd, None, out, lse, A, 1 / math.sqrt(3 * D), bias)
    nws = lib.dsa_fwd_workspace_bytes(ctypes.byref(a))
    ws = torch.zeros((nws,), dtype=torch.uint8, device=gpu)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nws
    _say(f"[order] B={B} L={L}")
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    _lib.check(lib.dsa_fwd(ctypes.byref(a), stream), "dsa_fwd")
    torch.cuda.synchronize(gpu)
    ntiles = (L + 127) // 128
    n = B * ntiles
    ints = ws[: 8 * n].view(torch.int32).cpu()
    cost, order = ints[:n].long(), ints[n:2 * n].long()
    want = _host_order_costs(seg, ntiles, per=2).reshape(-1)
    assert torch.equal(cost, want), "launch-order costs differ from the host count"
    assert torch.equal(torch.sort(order).values, torch.arange(n)), "the order is not a permutation of the items"
    assert bool((cost[order][1:] <= cost[order][:-1]).all()), "the order is not heaviest first"


def test_all_kept_key_mask_runs_as_no_mask(gpu):
    """A (B, 1, 1, L) key mask that keeps every key is recognised by an
    asynchronous device check (the first call starts it, no call waits):
    once it has finished, the mask runs as no mask, with results equal to the
    unmasked call's; a mask with one dropped key is never taken for one."""
    from deberta_amd.masks import kernel_masks

    B, L, H, D, A = 2, 256, 4, 64, 256
    g = torch.Generator().manual_seed(81)
    mk = lambda *s: torch.randn(*s, generator=g).to(gpu, torch.bfloat16)
    q, k, v, dout = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, 2 * A, D), mk(H, 2 * A, D)
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=gpu)
    ones = torch.ones(B, 1, 1, L, dtype=torch.bool, device=gpu)
    holes = ones.clone()
    holes[1, 0, 0, L - 1] = False
    kk, pk = kernel_masks(ones, B, L, L, gpu)  # starts the check
    assert kk is not None and pk is None
    kernel_masks(holes, B, L, L, gpu)
    torch.cuda.synchronize(gpu)
    assert kernel_masks(ones, B, L, L, gpu) == (None, None)
    kk, _ = kernel_masks(holes, B, L, L, gpu)
    assert kk is not None and int(kk.sum()) == B * L - 1
    # an integer mask handed over directly (as the reference's callers may):
    # the check is kept on the caller's tensor, not on its boolean copy
    ones_int = torch.ones(B, 1, 1, L, dtype=torch.int64, device=gpu)
    kernel_masks(ones_int, B, L, L, gpu)
    torch.cuda.synchronize(gpu)
    assert kernel_masks(ones_int, B, L, L, gpu) == (None, None)

    def run(kkm):
        leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, kr, qr)]
        out, _, _, _ = torch.ops.deberta_amd.dsa_fwd(*leaves, table, kkm, None, A, 1 / math.sqrt(3 * D))
        return [out] + list(torch.autograd.grad(out, leaves, dout))

    # the key-mask kernels on the all-kept mask give the unmasked results
    ref = run(None)
    got = run(ones.view(torch.uint8)[:, 0, 0, :])
    for name, a, b in zip(["out", "dq", "dk", "dv", "dkr", "dqr"], got, ref):
        if name in ("dkr", "dqr"):
            # bf16 roundings of fp32 sums taken in other orders (the masked
            # table kernel splits its items differently): one bf16 ulp
            err = float((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30))
            assert err <= 1e-2, f"{name}: {err:.3e}"
        else:
            assert torch.equal(a, b), f"{name}: the key-mask kernels differ from the unmasked ones"


@pytest.mark.parametrize("types", ["c2p|p2c", "c2p|p2c|p2p"])
def test_packed_qkv_op_equals_separate_op(types, gpu):
    """``deberta_amd::dsa_fwd_packed`` (q, k, v as one ``[B, L, 3, H, D]``
    tensor, its gradient returned as one tensor) gives the separate op's
    output and gradients: out and the q, k, v gradients bit for bit, the
    table gradients up to the order of their fp32 atomic additions."""
    from deberta_amd import ops
    from deberta_amd.attention import relative_operands

    B, L, H, D, A = 2, 320, 4, 64, 256
    g = torch.Generator().manual_seed(91)
    qkv0 = torch.randn(B, L, 3, H, D, generator=g).to(gpu, torch.bfloat16)
    kr0, qr0 = (torch.randn(H, 2 * A, D, generator=g).to(gpu, torch.bfloat16) for _ in range(2))
    dout = torch.randn(B, L, H, D, generator=g).to(gpu, torch.bfloat16)
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=gpu)
    scale = 1 / math.sqrt(D * (1 + len(types.split("|"))))
    tl = types.split("|")

    def run(packed):
        qkv = qkv0.detach().clone().requires_grad_(True)
        kr, qr = (t.detach().clone().requires_grad_(True) for t in (kr0, qr0))
        q, k, v = qkv.unbind(2)
        krx, qrx, qc = relative_operands(tl, q, kr, qr, A)
        if packed:
            out, _, _, _ = ops.attention_packed(qkv, krx, qrx, table, None, None, A, scale, True, qc)
        else:
            out, _, _, _ = ops.attention(q, k, v, krx, qrx, table, None, None, A, scale, True, qc)
        return [out] + list(torch.autograd.grad(out, [qkv, kr, qr], dout))

    _say(f"[packed] {types}")
    ref, got = run(False), run(True)
    for name, a, b in zip(["out", "dqkv", "dkr", "dqr"], got, ref):
        if name in ("dkr", "dqr"):
            err = float((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30))
            assert err <= 1e-2, f"{name}: {err:.3e}"  # bf16 roundings of fp32 sums in other orders
        else:
            assert torch.equal(a, b), f"{name} differs between the packed and the separate op"



@pytest.mark.parametrize("types", ["c2p", "p2c"])
def test_bias_api_casts_tables_to_query_dtype(types, gpu, monkeypatch):
    """The reference's dtype contract of the relative products
    (tests/test_smoke.py:1904-1965, :1968-2029) on the kernels: bf16
    projected tables meet float32 layers in float32 (tests/_modules.py
    ``bias_dtype_contract``; the CPU route has the same test in
    tests/test_module_cpu.py)."""
    from tests._modules import bias_dtype_contract

    err = bias_dtype_contract(types, gpu, monkeypatch)
    _say(f"[bias dtype contract {types}] rel {err:.2e}")
    assert err <= 1e-5
