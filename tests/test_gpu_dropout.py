"""Attention dropout in the fused kernels (deberta_v2_native.py:222, 636) on
the GPU, against the CPU oracle with the kernels' keep mask restated on the
CPU (oracle/dropout.py, pinned by Philox4x32-10's known-answer vectors).

* The keep bits themselves, bit for bit: with V one-hot over a block of 64
  keys, the fp32 output of query i at column j - 64 m is P_ij * scale when
  the pair is kept and exactly zero when it is dropped.
* The op's output and every gradient against the oracle with that mask
  (bf16 2e-2 absolute, fp32 1e-4 of scale): no mask, key, segment, pair and
  dead-row masks, D = 32 and 64, several probabilities, ragged lengths.
* The backward regenerates the forward's bits: the stage-split backward
  equals the one-call backward; the same seed gives bitwise equal results,
  another seed different ones.
* The module in training mode runs the kernels (not the torch path) and
  matches the oracle module given the mask of the seed it drew.
* The kept share over a large call is 1 - t / 65536 within its binomial
  spread.
"""

from __future__ import annotations

import ctypes
import functools
import math
import sys

import pytest
import torch

from oracle import eager
from oracle.dropout import keep_mask
from tests._cases import Case, max_rel
from tests._modules import _errors, _pair, _run
from tests.test_gpu_parity import _check

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _seed_t(seed: int) -> torch.Tensor:
    return torch.tensor([seed], dtype=torch.int64)


def _extract(B, H, L, t, seed, types, gpu):
    """The kernels' keep mask [B, H, L, L] read off fp32 outputs with V one-hot
    over each 64-key block, and the kept values (P * scale) beside it."""
    from deberta_amd.relpos import relative_offset_table

    D, A = 64, 256
    g = torch.Generator().manual_seed(seed & 0xFFFF)
    q = (torch.randn(B, L, H, D, generator=g) * 0.3).to(gpu)
    k = (torch.randn(B, L, H, D, generator=g) * 0.3).to(gpu)
    kr = (torch.randn(H, 2 * A, D, generator=g) * 0.3).to(gpu) if "c2p" in types else None
    qr = (torch.randn(H, 2 * A, D, generator=g) * 0.3).to(gpu) if "p2c" in types else None
    table = relative_offset_table(L, L, bucket_size=A, max_position=512, device=gpu) if types else None
    scale = 1.0 / math.sqrt(D * (1 + len(types)))
    kept = torch.zeros(B, H, L, L, dtype=torch.bool)
    vals = torch.zeros(B, H, L, L)
    for m in range((L + 63) // 64):
        v = torch.zeros(B, L, H, D)
        for j in range(64 * m, min(L, 64 * m + 64)):
            v[:, j, :, j - 64 * m] = 1.0
        out, _, _, _ = torch.ops.deberta_amd.dsa_fwd(
            q, k, v.to(gpu), kr, qr, table, None, None, A, scale, False, None, t, _seed_t(seed)
        )
        o = out.cpu().permute(0, 2, 1, 3)  # [B, H, L, D]
        n = min(L, 64 * m + 64) - 64 * m
        kept[..., 64 * m : 64 * m + n] = o[..., :n] != 0
        vals[..., 64 * m : 64 * m + n] = o[..., :n]
    # the probabilities without dropout, from the oracle
    rel = eager.relative_positions(L, L, A, 512) if types else None
    _, probs = eager.attend(
        q.cpu().permute(0, 2, 1, 3), k.cpu().permute(0, 2, 1, 3), torch.zeros(B, H, L, D), None if kr is None else kr.cpu(),
        None if qr is None else qr.cpu(), rel, None, types=list(types), att_span=A, use_relative=bool(types),
    )
    return kept, vals, probs


@pytest.mark.parametrize(
    "B,H,L,t,types",
    [(2, 3, 200, 6554, ("c2p", "p2c")), (1, 2, 130, 32768, ()), (1, 2, 64, 1, ()), (1, 1, 96, 65535, ("c2p",))],
)
def test_keep_bits_equal_the_contract(B, H, L, t, types, gpu):
    seed = 0x5EED_0000_0000_0001 + t
    _say(f"[dropout bits] B={B} H={H} L={L} t={t} types={types}")
    kept, vals, probs = _extract(B, H, L, t, seed, types, gpu)
    want = torch.from_numpy(keep_mask(seed, t, B, H, L, L))
    diff = int((kept != want).sum())
    _say(f"[dropout bits]   kept share {float(kept.float().mean()):.4f}, mismatches {diff}")
    assert diff == 0
    scale = 65536.0 / (65536 - t)
    err = float(((vals - probs * want * scale).abs() / (probs * scale).clamp(min=1e-30)).max())
    assert err <= 1e-4, err


@pytest.mark.parametrize(
    "c",
    [
        Case(B=2, H=4, L=256, D=64, dropout=0.1),
        Case(B=2, H=3, L=200, D=64, mask="key", dropout=0.1, seed=3),
        Case(B=1, H=2, L=300, D=64, mask="seg", dropout=0.3, seed=4),
        Case(B=1, H=2, L=192, D=64, mask="pair", dropout=0.1, seed=5),
        Case(B=1, H=2, L=130, D=32, dropout=0.2, seed=6),
        Case(B=2, H=3, L=130, D=64, types="", dropout=0.1, seed=7),
        Case(B=4, H=12, L=512, D=64, dropout=0.1, seed=12),
    ],
    ids=str,
)
def test_bf16_dropout(c, gpu):
    _check(c, torch.bfloat16, gpu)


@pytest.mark.parametrize(
    "c",
    [
        Case(B=1, H=2, L=300, D=64, dropout=0.1, seed=8),
        Case(B=2, H=2, L=128, D=32, mask="key", dropout=0.5, seed=9),
        Case(B=1, H=2, L=160, D=64, mask="dead", dropout=0.1, seed=10),
        Case(B=1, H=2, L=96, D=64, types="p2c", dropout=0.9, seed=11),
    ],
    ids=str,
)
def test_fp32_dropout(c, gpu):
    _check(c, torch.float32, gpu)


def _op_grads(q, k, v, kr, qr, table, A, scale, t, seed, dout):
    leaves = [x.detach().clone().requires_grad_(True) for x in (q, k, v, kr, qr)]
    out, _, _, _ = torch.ops.deberta_amd.dsa_fwd(*leaves, table, None, None, A, scale, True, None, t, _seed_t(seed))
    return [out.detach()] + [x.detach() for x in torch.autograd.grad(out, leaves, dout)]


def test_same_seed_same_result_other_seed_differs(gpu):
    from deberta_amd.relpos import relative_offset_table

    B, H, L, D, A = 2, 4, 256, 64, 256
    g = torch.Generator().manual_seed(2)
    q, k, v, dout = (torch.randn(B, L, H, D, generator=g).to(gpu, torch.bfloat16) for _ in range(4))
    kr, qr = (torch.randn(H, 2 * A, D, generator=g).to(gpu, torch.bfloat16) for _ in range(2))
    table = relative_offset_table(L, L, bucket_size=A, max_position=512, device=gpu)
    scale = 1.0 / math.sqrt(3 * D)
    a = _op_grads(q, k, v, kr, qr, table, A, scale, 6554, 77, dout)
    b = _op_grads(q, k, v, kr, qr, table, A, scale, 6554, 77, dout)
    c = _op_grads(q, k, v, kr, qr, table, A, scale, 6554, 78, dout)
    # out, dq, dk, dv bitwise (the table gradients sum with atomics)
    for x, y in zip(a[:4], b[:4]):
        assert torch.equal(x, y)
    assert all(max_rel(x.float().cpu(), y.float().cpu()) < 1e-2 for x, y in zip(a[4:], b[4:]))
    assert not torch.equal(a[0], c[0])


def test_backward_with_saved_or_regenerated_bits(gpu):
    """The backward given the forward's keep bits (dropout_bits), the
    backward that regenerates them from the seed in PREP, and the latter
    run as separate stage calls (PREP, DKDV, DQ|TABLE, SUM) give the same
    dq, dk, dv bit for bit and the same table gradients to their atomics'
    rounding."""
    from deberta_amd import _eager, _lib, ops
    from deberta_amd.relpos import relative_offset_table

    B, H, L, D, A = 2, 3, 200, 64, 256
    g = torch.Generator().manual_seed(4)
    q, k, v, dout = (torch.randn(B, L, H, D, generator=g).to(gpu, torch.bfloat16) for _ in range(4))
    kr, qr = (torch.randn(H, 2 * A, D, generator=g).to(gpu, torch.bfloat16) for _ in range(2))
    table = relative_offset_table(L, L, bucket_size=A, max_position=512, device=gpu)
    scale, t, seed = 1.0 / math.sqrt(3 * D), 13107, _seed_t(991)
    out, lse, bias, bits = torch.ops.deberta_amd.dsa_fwd(
        q, k, v, kr, qr, table, None, None, A, scale, True, None, t, seed
    )
    assert bits.numel() == ops.dropout_bytes(q, k, t)
    lib = _lib.load()
    stream = ctypes.c_void_p(_eager.stream_ptr(q))
    results = []
    split = [_lib.DSA_STAGE_PREP, _lib.DSA_STAGE_DKDV, _lib.DSA_STAGE_DQ | _lib.DSA_STAGE_TABLE, _lib.DSA_STAGE_SUM]
    for stages, saved in (([0], bits), ([0], None), (split, None)):
        grads = [torch.empty_like(x) for x in (q, k, v)]
        tabs = [torch.empty(H, 2 * A, D, device=gpu, dtype=torch.bfloat16) for _ in range(2)]
        a = ops.fill_bwd_args(dout, q, k, v, kr, qr, table, None, None, out, lse, bias, A, scale, *grads, *tabs,
                              dtab_overwrite=True, dropout_t=t, dropout_seed=seed, dropout_bits=saved)
        ws = torch.empty(ops.bwd_workspace_bytes(a), dtype=torch.uint8, device=gpu)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        for s in stages:
            a.stages = s
            _lib.check(lib.dsa_bwd(ctypes.byref(a), stream), "dsa_bwd")
        torch.cuda.synchronize()
        results.append([x.float().cpu() for x in grads + tabs])
    for other in results[1:]:
        for n, (x, y) in enumerate(zip(results[0], other)):
            if n < 3:
                assert torch.equal(x, y), n
            else:
                assert max_rel(x, y) < 1e-2, n


def test_static_forward_refuses_dropout(gpu):
    from deberta_amd import _eager, _lib, ops
    from deberta_amd.relpos import relative_offset_table

    B, H, L, D, A = 1, 2, 64, 64, 256
    q = torch.randn(B, L, H, D, device=gpu, dtype=torch.bfloat16)
    kr = torch.randn(H, 2 * A, D, device=gpu, dtype=torch.bfloat16)
    table = relative_offset_table(L, L, bucket_size=A, max_position=512, device=gpu)
    out = torch.empty_like(q)
    lse = torch.empty(B, H, L, device=gpu)
    a = ops._fill_fwd_args(q, q, q, kr, None, table, None, None, out, lse, A, 0.1, None, None, 6554, _seed_t(1))
    lib = _lib.load()
    assert lib.dsa_fwd_static(ctypes.byref(a), ctypes.c_void_p(_eager.stream_ptr(q))) != 0
    assert b"dropout" in lib.dsa_last_error()


def test_kept_share_matches_threshold(gpu):
    B, H, L, t = 2, 2, 512, 6554
    kept, _, _ = _extract(B, H, L, t, 0xC0FFEE, (), gpu)
    n = kept.numel()
    q = t / 65536
    sigma = math.sqrt(q * (1 - q) / n)
    share = 1 - float(kept.float().mean())
    _say(f"[dropout share] dropped {share:.5f} want {q:.5f} (sigma {sigma:.1e})")
    assert abs(share - q) <= 6 * sigma


@pytest.mark.parametrize("share", [False, True])
def test_module_training_dropout_runs_in_the_kernels(share, gpu, monkeypatch):
    """DisentangledSelfAttention in training mode with attention dropout 0.1
    (the HF preset): the fused kernels run (the torch path is switched off
    for the test) and the output and every gradient equal the oracle module
    given the mask of the seed the module drew (fp32, 1e-4 of scale)."""
    import deberta_amd.attention as att
    from deberta_amd import ops

    def _no_torch_path(*a, **k):
        raise AssertionError("the torch path ran")

    monkeypatch.setattr(att, "unfused_attention", _no_torch_path)
    cfg = eager.make_config(
        hidden_size=128, num_attention_heads=4, position_buckets=256, max_relative_positions=512,
        share_att_key=share, attention_probs_dropout_prob=0.1, hidden_dropout_prob=0.0,
    )
    ref, ours = _pair(cfg)
    ours = ours.to(gpu).train()
    B, L = 2, 160
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, L, 128, generator=g)
    rel = torch.randn(512, 128, generator=g) * 0.02
    keep = torch.ones(B, L, dtype=torch.bool)
    keep[1, 101:] = False
    m = keep[:, None, None, :]
    torch.manual_seed(2024)
    b = _run(ours, x, m, rel, gpu)
    torch.manual_seed(2024)
    seed = int(ops.draw_dropout_seed())
    t = ops.dropout_threshold(0.1)
    kmask = torch.from_numpy(keep_mask(seed, t, B, 4, L, L))
    ref.forward = functools.partial(ref.forward, dropout_keep=kmask, dropout_p=t / 65536)
    a = _run(ref, x, m, rel, "cpu")
    errs = _errors(a, b)
    _say(f"[module dropout share={share}] {errs}")
    assert all(e <= 1e-4 for e in errs.values()), errs


@pytest.mark.parametrize("backend", ["aot_eager", "inductor"])
def test_module_dropout_under_compile(backend, gpu):
    """Training-mode attention dropout inside torch.compile: the seed is
    drawn inside the compiled region.  aot_eager draws it as eager does, so
    with the same manual seed the compiled output equals the eager one bit
    for bit and the gradients agree; inductor draws with its own generator,
    so its result is checked by repeatability (same manual seed, same
    output), by a new seed changing it, and by the gradients being finite."""
    torch._dynamo.reset()
    cfg = eager.make_config(
        hidden_size=256, num_attention_heads=4, share_att_key=True, attention_probs_dropout_prob=0.1,
        hidden_dropout_prob=0.0,
    )
    _, ours = _pair(cfg, seed=5)
    ours = ours.to(gpu).train()
    x = torch.randn(2, 256, 256, device=gpu)
    rel = torch.randn(512, 256, device=gpu)

    def run(mod, seed):
        torch.manual_seed(seed)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out, _ = mod(x, None, rel_embeddings=rel)
        loss = out.float().square().mean()
        return out.detach(), torch.autograd.grad(loss, list(ours.parameters()))

    compiled = torch.compile(ours, backend=backend, dynamic=False)
    oc1, gc1 = run(compiled, 11)
    oc2, _ = run(compiled, 11)
    oc3, _ = run(compiled, 12)
    assert torch.equal(oc1, oc2) and not torch.equal(oc1, oc3)
    assert all(torch.isfinite(g).all() for g in gc1)
    if backend == "aot_eager":
        oe, ge = run(ours, 11)
        assert torch.equal(oe, oc1)
        for a, b in zip(ge, gc1):
            assert max_rel(b.float().cpu(), a.float().cpu()) <= 1e-2
