"""dsa_fwd_static, the forward entry point that allocates nothing: its
launch-order scratch is a library-owned static device array (no
counterpart in the reference; for callers that cannot allocate).  Its
results equal dsa_fwd's with a caller workspace, call after call, and sizes
beyond the array are refused before any device work."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from deberta_amd import _lib, ops
from deberta_amd.masks import SegmentMask, kernel_masks
from deberta_amd.relpos import relative_offset_table


def _forward(entry, q, k, v, kr, qr, table, kk, pk, A, scale):
    B, Lq, H, D = q.shape
    out = torch.empty_like(q)
    lse = torch.empty((B, H, Lq), dtype=torch.float32, device=q.device)
    # zero-filled: under key or segment masks the forward writes the saved
    # term only for the key tiles it visits (the backward reads no others)
    bias = torch.zeros(ops.bias_shape(q, k), dtype=ops.bias_dtype(q.dtype), device=q.device)
    a = ops._fill_fwd_args(q, k, v, kr, qr, table, kk, pk, out, lse, A, scale, bias)
    lib = _lib.load()
    ws = None
    if entry == "dsa_fwd":
        n = lib.dsa_fwd_workspace_bytes(ctypes.byref(a))
        if n:
            ws = torch.empty((n,), dtype=torch.uint8, device=q.device)
            a.workspace, a.workspace_bytes = ws.data_ptr(), n
    stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
    _lib.check(getattr(lib, entry)(ctypes.byref(a), stream), entry)
    torch.cuda.synchronize(q.device)
    return out, lse, bias


def _inputs(B, L, H, D, mask, seed, dev):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(dev, torch.bfloat16)
    q, k, v = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, 512, D), mk(H, 512, D)
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=dev)
    if mask == "key":
        lens = torch.randint(L // 4, L + 1, (B,), generator=g)
        m = (torch.arange(L)[None, :] < lens[:, None])[:, None, None, :].to(dev)
    else:
        ids = (torch.arange(L)[None, :] // 97 + torch.arange(B)[:, None]) % 5 + 1
        ids[:, L - L // 7:] = 0
        m = SegmentMask(ids.to(dev))
    kk, pk = kernel_masks(m, B, L, L, dev)
    return q, k, v, kr, qr, table, kk, pk


@pytest.mark.gpu
def test_static_forward_equals_the_workspace_forward(gpu):
    """Two calls in a row, the second smaller, each against dsa_fwd with a
    caller workspace: out, lse and the saved relative term bit for bit."""
    A, scale = 256, 1.0 / math.sqrt(64 * 3)
    for B, L, H, mask, seed in ((4, 700, 4, "key", 0), (2, 300, 2, "seg", 1)):
        x = _inputs(B, L, H, 64, mask, seed, gpu)
        want = _forward("dsa_fwd", *x, A, scale)
        got = _forward("dsa_fwd_static", *x, A, scale)
        for name, a_, b_ in zip(("out", "lse", "bias"), got, want):
            assert torch.equal(a_, b_), (B, L, mask, name)


def test_static_forward_refuses_sizes_past_its_scratch():
    """B * ceil(Lq / 128) launch-order items beyond the 512 KiB array are
    refused with an error, before any device work."""
    lib = _lib.load()
    a = _lib.DsaFwdArgs()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p).value
    for f in ("q", "k", "v", "out", "lse", "key_keep"):
        setattr(a, f, p)
    a.B, a.H, a.Lq, a.Lk, a.D, a.dtype = 65535, 1, 256, 256, 64, _lib.DSA_BF16
    assert lib.dsa_fwd_static(ctypes.byref(a), None) != 0
    assert "exceed the static scratch" in _lib.last_error()
