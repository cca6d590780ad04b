"""Configurations 2 and 4 at their full sizes, through properties that hold
at any size (the CPU oracle is too slow at these shapes; the oracle
comparisons of the same code paths run at smaller sizes in
test_gpu_parity.py).

* Configuration 2 (B=32, L=512, H=12, D=64, bf16, key padding with valid
  lengths uniform in [64, 512]): each batch row of the padded run equals the
  same row run alone at its valid length without a mask, and the padded keys
  get exactly zero gradient.  The upstream gradient of padded query rows is
  zero, so that they contribute nothing (they attend the valid keys, as in
  the reference, whose key-padding mask leaves them live).
* Configuration 2 in the encoder's pair form (keep_i & keep_j): its live
  rows and every key's gradients equal the key-mask run's with the padded
  rows' upstream gradient zeroed; dead rows give exact zeros.
* Configuration 4 (B=4, L=4096, H=12, D=64, bf16, packed documents given as
  segment ids; lengths as in the configuration but at least 96 tokens):
  each document of the packed run equals the document run alone as its own
  sequence (the relative position of two tokens of one document is the same
  in both; pairs across documents are masked).

Outputs and input gradients are compared element by element with max|err|
<= 2e-2 * max(1, max|ref|) (bf16 results of different tile partitions;
the padded rows of configuration 2 use the same partitions and come out
equal in practice); the relative-table gradients against the sum of the
separate runs' with max|err| / max|ref| <= 1e-2 (fp32 atomic sums of bf16
dS values in different orders).
"""

from __future__ import annotations

import math
import sys

import pytest
import torch

from deberta_amd.masks import SegmentMask, kernel_masks
from deberta_amd.relpos import relative_offset_table

pytestmark = pytest.mark.gpu

H, D, A = 12, 64, 256
MIN_DOC = 96  # shortest document of configuration 4 here (shortest sequence of the GPU parity cases)


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _run(q, k, v, kr, qr, dout, mask):
    """Fused fwd + bwd; returns out, dq, dk, dv, dkr, dqr (fp32)."""
    B, L = q.shape[:2]
    dev = q.device
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v, kr, qr)]
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=dev)
    kk, pk = kernel_masks(mask, B, L, L, dev) if mask is not None else (None, None)
    out, _, _, _ = torch.ops.deberta_amd.dsa_fwd(*leaves, table, kk, pk, A, 1.0 / math.sqrt(3 * D))
    grads = torch.autograd.grad(out, leaves, dout)
    return [out.detach().float()] + [g.float() for g in grads]


def _inputs(B, L, seed, dev):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(dev, torch.bfloat16)
    return mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D), mk(H, 2 * A, D), mk(H, 2 * A, D), mk(B, L, H, D), g


def _close(name, got, ref):
    err = float((got - ref).abs().max()) if ref.numel() else 0.0
    tol = 2e-2 * max(1.0, float(ref.abs().max()) if ref.numel() else 1.0)
    assert err <= tol, f"{name}: max|err| {err:.3e} > {tol:.3e}"


def _tables(name, got, ref):
    err = float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
    assert err <= 1e-2, f"{name}: max|err| / max|ref| = {err:.3e}"


def test_config2_padded_rows_equal_unpadded_runs(gpu):
    B, L = 32, 512
    q, k, v, kr, qr, dout, g = _inputs(B, L, 61, gpu)
    lens = torch.randint(64, L + 1, (B,), generator=g)
    keep = torch.arange(L)[None, :] < lens[:, None]
    dout = dout * keep[:, :, None, None].to(gpu, dout.dtype)  # padded query rows: no upstream gradient
    _say(f"[fullsize] C2 padded B={B} L={L}, lengths {int(lens.min())}..{int(lens.max())}")
    out, dq, dk, dv, dkr, dqr = _run(q, k, v, kr, qr, dout, keep[:, None, None, :].to(gpu))
    sum_kr = torch.zeros_like(dkr)
    sum_qr = torch.zeros_like(dqr)
    for b in range(B):
        n = int(lens[b])
        sl = lambda t: t[b : b + 1, :n]
        r = _run(sl(q), sl(k), sl(v), kr, qr, sl(dout), None)
        for name, got, ref in zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv), r[:4]):
            _close(f"row {b} {name}", got[b : b + 1, :n], ref)
        assert float(dk[b, n:].abs().max() if n < L else 0.0) == 0.0, f"row {b}: padded keys got a dk"
        assert float(dv[b, n:].abs().max() if n < L else 0.0) == 0.0, f"row {b}: padded keys got a dv"
        sum_kr += r[4]
        sum_qr += r[5]
    _tables("dkr", dkr, sum_kr)
    _tables("dqr", dqr, sum_qr)


def test_config2_pair_form_equals_key_form_on_live_rows(gpu):
    """Configuration 2's padding as the reference's encoder hands it to its
    layers (get_attention_mask, deberta_v2_native.py:1049-1068: the pair
    mask keep_i & keep_j, padded queries dead rows; recognised and run as
    segment ids) against the key-mask run of the same inputs whose padded
    query rows get no upstream gradient: live rows and every key's
    gradients agree, dead rows' outputs and dq are exactly zero, and the
    dead rows' upstream gradient (left nonzero here) reaches nothing."""
    B, L = 32, 512
    q, k, v, kr, qr, dout, g = _inputs(B, L, 62, gpu)
    lens = torch.randint(64, L + 1, (B,), generator=g)
    keep = torch.arange(L)[None, :] < lens[:, None]
    pair = (keep[:, :, None] & keep[:, None, :])[:, None].to(gpu)
    kk, pk = kernel_masks(pair, B, L, L, gpu)
    assert pk is None and kk is not None and kk.dtype == torch.int32, "padding pair mask not run as segments"
    _say(f"[fullsize] C2 pair form B={B} L={L}, lengths {int(lens.min())}..{int(lens.max())}")
    got = _run(q, k, v, kr, qr, dout, pair)
    live = keep[:, :, None, None].to(gpu)
    ref = _run(q, k, v, kr, qr, dout * live.to(dout.dtype), keep[:, None, None, :].to(gpu))
    for name, a, b in zip(("out", "dq"), got[:2], ref[:2]):
        _close(f"live rows {name}", a * live, b * live)
        assert float((a * ~live).abs().max()) == 0.0, f"dead rows: nonzero {name}"
    for name, a, b in zip(("dk", "dv"), got[2:4], ref[2:4]):
        _close(name, a, b)
        assert float((a * ~live).abs().max()) == 0.0, f"padded keys got a {name}"
    _tables("dkr", got[4], ref[4])
    _tables("dqr", got[5], ref[5])


def test_config4_packed_documents_equal_separate_runs(gpu):
    B, L = 4, 4096
    q, k, v, kr, qr, dout, g = _inputs(B, L, 62, gpu)
    ids = torch.zeros(B, L, dtype=torch.int64)
    spans = []
    for r in range(B):  # document lengths 1 + Geometric(p = 1/600), cut at the row's end
        pos, doc = 0, 1
        while pos < L:
            u = float(torch.rand((), generator=g, dtype=torch.float64))
            n = min(1 + int(math.floor(math.log1p(-u) / math.log1p(-1.0 / 600.0))), L - pos)
            # at least MIN_DOC tokens (the separate runs' shortest sequence);
            # a shorter tail joins the row's last document
            n = max(n, min(MIN_DOC, L - pos))
            if L - pos - n < MIN_DOC:
                n = L - pos
            ids[r, pos : pos + n] = doc
            spans.append((r, pos, pos + n))
            pos, doc = pos + n, doc + 1
    _say(f"[fullsize] C4 packed B={B} L={L}, {len(spans)} documents")
    out, dq, dk, dv, dkr, dqr = _run(q, k, v, kr, qr, dout, SegmentMask(ids.to(gpu)))
    sum_kr = torch.zeros_like(dkr)
    sum_qr = torch.zeros_like(dqr)
    for r, s, e in spans:
        sl = lambda t: t[r : r + 1, s:e]
        ref = _run(sl(q), sl(k), sl(v), kr, qr, sl(dout), None)
        for name, got, want in zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv), ref[:4]):
            _close(f"doc ({r}, {s}:{e}) {name}", got[r : r + 1, s:e], want)
        sum_kr += ref[4]
        sum_qr += ref[5]
    _tables("dkr", dkr, sum_kr)
    _tables("dqr", dqr, sum_qr)
