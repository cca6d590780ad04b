"""Benchmark of the fused disentangled-attention forward + backward on one
MI355X, in the shape the headline metric is quoted on (BASELINE.json
configs[1], all-ones mask): B=32, L=512, H=12, D=64, bf16, position buckets
256, max relative positions 512, c2p|p2c.

A step is one forward and one backward of the op on leaf tensors already
resident in HBM (q, k, v [B, L, H, D]; projected relative tables kr, qr
[H, 512, D]; upstream gradient dO).  Projections are outside the op and
outside the timed region.  The algorithmic count is
  F_fwd = 4 B H D L^2 + 4 B H D L R,   F_step = 3 F_fwd,   R = 2A = 512.

Prints one JSON line (rank 0) with the throughput, the roofline of the
dominant kernel (per-kernel times from HIP events on the launch stream),
and the CPU baseline: the fp32 eager oracle timed on this host's cores on a
bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "disentangled-attn fwd+bwd TFLOP/s & % bf16 MFMA peak, L=512 H=12 d=64"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (published 2.5 PFLOP/s)
B, L, H, D, BUCKETS, MAX_POS = 32, 512, 12, 64, 256, 512
A = BUCKETS
R = 2 * A

# --workload: the headline (default) and the other BASELINE shapes that fit
# one GPU, for reference figures; only the headline's line is the metric.
#   name: (batch, seq_len, heads, mask kind, description)
WORKLOADS = {
    "headline": (32, 512, 12, None, "BASELINE configs[1] shape, all-ones mask"),
    "C2pad": (32, 512, 12, "pad", "configs[1] shape, per-row valid length ~U{64..512}, given as the encoder gives a padding mask to its layers: the (B,1,L,L) pair mask keep_i & keep_j (recognised once and run as segment ids)"),
    "C2key": (32, 512, 12, "key", "as C2pad, the same lengths as a (B,1,1,L) key mask: every query row, padded ones included, attends to its row's valid keys"),
    "C5": (64, 512, 16, None, "B=64 L=512 H=16, no mask"),
    "C3": (16, 512, 12, None, "12-layer DeBERTa-v3-base-shaped encoder fwd+bwd under an RTD loss, bf16 autocast, fused attention and fused row kernels around it (step time with plain torch blocks beside it)"),
    "C5layer": (64, 512, 16, None, "DeBERTa-v3-large-shaped attention layer (hidden 1024, projections included) fwd+bwd, bf16, inside torch.compile"),
    "C4": (4, 4096, 12, "doc", "B=4 L=4096 H=12, packed documents (lengths ~Geometric(mean 600)) as the dense (B,1,L,L) doc-block mask (recognised once and run as segment ids)"),
    "C4seg": (4, 4096, 12, "seg", "as C4, the same documents given as segment ids (SegmentMask)"),
    "plain": (32, 512, 12, None, "headline shape without relative terms, beside torch's scaled_dot_product_attention (flash backend)"),
    "eager": (32, 512, 12, None, "headline op fwd+bwd beside the reference's op chain in torch operations on the same GPU (deberta_amd.unfused: float32 scores and relative terms, gathers, softmax, value product)"),
}


# untimed op steps between the per-kernel timing and the W warm-up steps
SETTLE_STEPS = 400

# HBM bytes per launch at this workload come from the committed rocprofv3
# summary of this build's kernels (two --pmc passes over `bench.py
# --kernels-only`, FETCH_SIZE then WRITE_SIZE in KiB per dispatch, each
# scaled by what the counter reads for a plain device copy of known size in
# the same run; commands, raw figures and factors in the file).
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_headline.md")


def traffic_table(path: str = TRAFFIC_PROFILE):
    """{kernel: (FETCH_SIZE KiB, WRITE_SIZE KiB)} and the two scale factors,
    parsed from the profile summary's table and its calibration sentence
    ("FETCH_SIZE is scaled by F and WRITE_SIZE by W")."""
    import re

    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return {}, None, None
    rows = {}
    for m in re.finditer(r"^\| (dsa_\w+) \| (\d+) \| (\d+) \|", text, re.M):
        rows[m.group(1)] = (int(m.group(2)), int(m.group(3)))
    m = re.search(r"FETCH_SIZE is scaled by ([0-9.]+) and WRITE_SIZE by ([0-9.]+)", text)
    if not m:
        return rows, None, None
    return rows, float(m.group(1)), float(m.group(2))


def hbm_bytes(stage: str):
    """HBM bytes per launch of a bench stage (the sum over its kernels), or
    None when the profile does not cover them."""
    rows, fs, ws = traffic_table()
    names = [k for k in rows if k in stage]
    if not names or fs is None:
        return None
    return int(round(sum(rows[k][0] * fs + rows[k][1] * ws for k in names) * 1024))


def mfma_peak_probe(dev) -> dict:
    """Measured bf16 dense MFMA throughput of this GPU (libdsa_probe.so:
    four independent v_mfma_f32_32x32x16_bf16 chains per wave, eight
    workgroups of four waves per CU), timed with HIP events on its stream:
    the measured figure beside the published 2.5 PFLOP/s."""
    import ctypes

    import torch

    from deberta_amd._build import PROBE_PATH

    lib = ctypes.CDLL(str(PROBE_PATH))
    lib.dsa_probe_mfma_bf16.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.dsa_probe_mfma_bf16.restype = ctypes.c_int
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    wgs, iters = 8 * cus, 2048
    sink = torch.empty(wgs * 256, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev)
    run = lambda: lib.dsa_probe_mfma_bf16(wgs, iters, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(st.cuda_stream))
    for _ in range(3):
        if run():
            raise RuntimeError("MFMA probe launch failed")
    best = float("inf")
    for _ in range(5):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        run()
        b.record(st)
        torch.cuda.synchronize(dev)
        best = min(best, a.elapsed_time(b))
    flops = wgs * 4.0 * iters * 4 * 32768
    return {"tflops": round(flops / (best * 1e-3) / 1e12, 1), "cus": cus, "workgroups": wgs, "ms": round(best, 4)}


def dsfree_flush_probe(dev, B: int, H: int, L: int) -> dict:
    """Time of the fp32 atomic traffic that a backward without its dS
    workspace would make to reduce the relative-table gradients over the
    batch (libdsa_probe.so: one workgroup per (b, h, 128-key tile) adding
    one 64-float row per offset its keys meet and per kind, after summing
    its four waves), beside the bytes of dS's own round trip."""
    import ctypes

    import torch

    from deberta_amd._build import PROBE_PATH

    lib = ctypes.CDLL(str(PROBE_PATH))
    lib.dsa_probe_dsfree_flush.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.dsa_probe_dsfree_flush.restype = ctypes.c_int
    acc = torch.zeros(H * 2 * 2 * L * 64, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev)
    run = lambda: lib.dsa_probe_dsfree_flush(B, H, L, ctypes.c_void_p(acc.data_ptr()), ctypes.c_void_p(st.cuda_stream))
    for _ in range(3):
        if run():
            raise RuntimeError("atomics probe launch failed")
    ms = []
    for _ in range(10):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        run()
        b.record(st)
        torch.cuda.synchronize(dev)
        ms.append(a.elapsed_time(b))
    ms.sort()
    nbytes = B * H * (L // 128) * 2 * (L + 127) * 256
    med = ms[len(ms) // 2]
    return {
        "workload": f"B={B} H={H} L={L}",
        "atomic_bytes": nbytes,
        "ms_median": round(med, 4),
        "tb_per_s": round(nbytes / (med * 1e-3) / 1e12, 3),
        "ds_round_trip_bytes": B * H * L * L * 2 * 2,
    }


class HipEvents:
    """HIP timing events without the system-scope fence (the runtime's
    hipEventDisableSystemFence flag): torch's events write back and
    invalidate the caches when recorded, which leaves a gap of about 6 us
    before the next kernel and slows it, so an event between every two
    kernels would inflate each kernel's time.  These only timestamp the
    stream; nothing reads data through them."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, n: int):
        self.rt = ctypes.CDLL("libamdhip64.so")  # the runtime torch has loaded
        self.rt.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.rt.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            if self.rt.hipEventCreateWithFlags(ctypes.byref(e), self.DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            self.ev.append(e)

    def record(self, i: int, stream_ptr: int) -> None:
        if self.rt.hipEventRecord(self.ev[i], ctypes.c_void_p(stream_ptr)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def ms(self, i: int, j: int) -> float:
        """Milliseconds from event i to event j (both complete)."""
        t = ctypes.c_float()
        if self.rt.hipEventElapsedTime(ctypes.byref(t), self.ev[i], self.ev[j]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return t.value

    def __del__(self):
        for e in getattr(self, "ev", []):
            self.rt.hipEventDestroy(e)


def flops_fwd(b: int, l: int, h: int, d: int, r: int) -> float:
    return 4.0 * b * h * d * l * l + 4.0 * b * h * d * l * r


def workload_mask(kind, b: int, l: int, g, dev):
    """Synthetic mask of a workload, drawn from the generator g.

    Returns (attention_mask, kept pairs, live query rows)."""
    import torch

    from deberta_amd.masks import SegmentMask, build_doc_block_mask

    if kind is None:
        return None, b * l * l, b * l
    if kind in ("key", "pad"):
        lens = torch.randint(64, l + 1, (b,), generator=g)
        keep = torch.arange(l)[None, :] < lens[:, None]
        if kind == "key":  # every query row attends to the row's valid keys
            return keep[:, None, None, :].to(dev), l * int(lens.sum()), b * l
        # the encoder's form of a padding mask (deberta_v2_native.py:1049-1068):
        # padded query rows keep no key
        pair = keep[:, :, None] & keep[:, None, :]
        return pair[:, None].to(dev), int((lens.double() ** 2).sum()), int(lens.sum())
    ids = torch.zeros(b, l, dtype=torch.int64)
    for r in range(b):  # document lengths 1 + Geometric(p = 1/600) by inversion, cut at the row's end
        pos, doc = 0, 1
        while pos < l:
            u = float(torch.rand((), generator=g, dtype=torch.float64))
            n = 1 + int(math.floor(math.log1p(-u) / math.log1p(-1.0 / 600.0)))
            n = min(n, l - pos)
            ids[r, pos : pos + n] = doc
            pos, doc = pos + n, doc + 1
    dense = build_doc_block_mask(ids)
    kept = int(dense.sum())
    if kind == "doc":
        return dense[:, None].to(dev), kept, b * l
    return SegmentMask(ids.to(dev)), kept, b * l


def run_encoder(args) -> None:
    """C3: a 12-layer DeBERTa-v3-base-shaped encoder (hidden 768, 12 heads,
    FFN 3072, vocab 128100, relative embeddings shared by the layers with a
    LayerNorm, keys shared with the relative projections) with the fused
    attention module in every layer, fwd+bwd of an RTD-style discriminator
    loss (BCE over a Bernoulli(0.15) replaced-token label per token) under
    bf16 autocast, on synthetic token ids, random init N(0, 0.02).  This is
    a measurement harness around the attention path, not a model of this
    package.  Prints step time, tokens/s and the attention share (the fused
    op's fwd+bwd at the same shape, times 12, over the step)."""
    import torch

    import deberta_amd
    from deberta_amd import ops
    from deberta_amd.relpos import relative_offset_table
    # The encoder is test code shared with the C3 GPU tests; only this
    # workload imports it (tests/ resolves as a namespace package from the
    # repository root, bench.py's directory).
    from tests._encoder import Encoder, init_weights, synthetic_batch

    dev = torch.device("cuda:0")
    Bc, Lc, Hc = 16, 512, 12
    ids, labels = synthetic_batch(Bc, Lc, seed=0)
    ids, labels = ids.to(dev), labels.to(dev)
    mask = torch.ones(Bc, 1, 1, Lc, dtype=torch.bool, device=dev)
    rel_pos = deberta_amd.build_relative_position(Lc, Lc, bucket_size=BUCKETS, max_position=MAX_POS, device=dev)

    def make_step(fused_blocks):
        model = Encoder(deberta_amd.DisentangledSelfAttention, fused_blocks=fused_blocks)
        init_weights(model, seed=0)
        model = model.to(dev)
        params = [p_ for p_ in model.parameters()]

        def step():
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss, _ = model.loss(ids, mask, rel_pos, labels)
            torch.autograd.grad(loss, params)

        return step

    def timed(fn, n):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    def timed_pair(fa, fb, n):
        """Median step times of two step functions run alternately (one
        step of each per round, each bracketed by events), so that clock
        and thermal drift fall on both alike."""
        for _ in range(3):
            fa()
            fb()
        torch.cuda.synchronize()
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n)]
        for e in ev:
            e[0].record()
            fa()
            e[1].record()
            e[2].record()
            fb()
            e[3].record()
        torch.cuda.synchronize()
        ta = sorted(e[0].elapsed_time(e[1]) for e in ev)
        tb = sorted(e[2].elapsed_time(e[3]) for e in ev)
        return ta[n // 2], tb[n // 2]

    n = max(3, args.steps)
    ms, ms_plain = timed_pair(make_step(True), make_step(False), n)
    # the fused op alone at one layer's shape (q, k, v, kr, qr leaves, bf16)
    gq = torch.Generator().manual_seed(1)
    mk = lambda *sh: torch.randn(*sh, generator=gq).to(device=dev, dtype=torch.bfloat16).requires_grad_(True)
    q, k, v = mk(Bc, Lc, Hc, D), mk(Bc, Lc, Hc, D), mk(Bc, Lc, Hc, D)
    kr, qr = mk(Hc, R, D), mk(Hc, R, D)
    dout = torch.randn(Bc, Lc, Hc, D, generator=gq).to(device=dev, dtype=torch.bfloat16)
    table = relative_offset_table(Lc, Lc, bucket_size=BUCKETS, max_position=MAX_POS, device=dev)
    scale = 1.0 / math.sqrt(D * 3)

    def attn_step():
        out, _, _, _ = ops.attention(q, k, v, kr, qr, table, None, None, A, scale)
        torch.autograd.grad(out, (q, k, v, kr, qr), dout)

    ms_attn = timed(attn_step, 10)
    print(
        json.dumps(
            {
                "workload": "C3",
                "description": WORKLOADS["C3"][4],
                "ms_per_step": round(ms, 3),
                "tokens_per_s": round(Bc * Lc / (ms * 1e-3), 1),
                "ms_per_step_plain_torch_blocks": round(ms_plain, 3),
                "timing": "median step of each, the two encoders stepped alternately",
                "attention_ms_per_layer": round(ms_attn, 4),
                "attention_share": round(12 * ms_attn / ms, 4),
                "steps": n,
                "data": "synthetic token ids and labels, random init",
            }
        ),
        flush=True,
    )


def run_plain(args) -> None:
    """The headline shape without relative terms (plain softmax attention,
    scale 1/sqrt(D)): the op's forward and fwd+bwd beside torch's
    scaled_dot_product_attention with the flash backend (bf16, (B, H, L, D)
    contiguous inputs), each timed over 50 launches after 300 warm-up ones.
    A reference figure for the kernels' attention machinery without the
    disentangled terms, not the metric."""
    import torch
    import torch.nn.functional as F

    import deberta_amd  # noqa: F401
    from deberta_amd import ops

    dev = torch.device("cuda:0")
    B, L, H, _, desc = WORKLOADS["plain"]
    g = torch.Generator(device="cpu").manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(device=dev, dtype=torch.bfloat16)
    q, k, v, dout = (mk(B, L, H, D) for _ in range(4))
    scale = 1.0 / math.sqrt(D)

    def timed(fn, n=50):
        for _ in range(300):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]

    def ours_step():
        out, _, _, _ = ops.attention(*leaves, None, None, None, None, None, 1, scale)
        torch.autograd.grad(out, leaves, dout)

    res = {
        "ours_fwd_ms": timed(lambda: ops.attention(q, k, v, None, None, None, None, None, 1, scale)),
        "ours_fwd_bwd_ms": timed(ours_step),
    }
    qh, kh, vh, dh = (t.permute(0, 2, 1, 3).contiguous() for t in (q, k, v, dout))
    sl = [t.detach().clone().requires_grad_(True) for t in (qh, kh, vh)]
    flash = torch.nn.attention.SDPBackend.FLASH_ATTENTION

    def sdpa_fwd():
        with torch.nn.attention.sdpa_kernel(flash):
            return F.scaled_dot_product_attention(qh, kh, vh)

    def sdpa_step():
        with torch.nn.attention.sdpa_kernel(flash):
            o = F.scaled_dot_product_attention(*sl)
        torch.autograd.grad(o, sl, dh)

    res["sdpa_flash_fwd_ms"] = timed(sdpa_fwd)
    res["sdpa_flash_fwd_bwd_ms"] = timed(sdpa_step)
    f = 4.0 * B * H * D * L * L  # QK^T and PV
    out = {"workload": "plain", "description": desc}
    for key, ms in res.items():
        fl = 3 * f if "bwd" in key else f
        out[key] = round(ms, 4)
        out[key.replace("_ms", "_tflops")] = round(fl / (ms * 1e-3) / 1e12, 1)
    print(json.dumps(out), flush=True)


def run_eager(args) -> None:
    """The headline fwd+bwd of the fused op beside the same attention as the
    reference computes it, in torch operations on the GPU (the package's
    torch path, deberta_amd.unfused: the reference's score chain of
    deberta_v2_native.py:592-652 with the dynamic bias of :349-432), both on
    the same bf16 leaves, or float32 ones with --fp32 (the reference's
    train.mixed_precision=no) (the fused op over 50 steps after 300 warm-up
    ones, the eager chain over 20 after 10: each warm-up is over 0.1 s).  A
    reference figure (the eager path's speed on this GPU), not the metric."""
    import torch

    import deberta_amd  # noqa: F401
    from deberta_amd import ops
    from deberta_amd.relpos import build_relative_position, relative_offset_table
    from deberta_amd.unfused import unfused_attention

    dev = torch.device("cuda:0")
    B, L, H, _, desc = WORKLOADS["eager"]
    # --fp32: both in float32, the reference's train.mixed_precision=no
    dtype = torch.float32 if args.fp32 else torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(device=dev, dtype=dtype)
    leaves = [mk(B, L, H, D) for _ in range(3)] + [mk(H, R, D) for _ in range(2)]
    for t in leaves:
        t.requires_grad_(True)
    dout = mk(B, L, H, D)
    scale = 1.0 / math.sqrt(D * 3)
    table = relative_offset_table(L, L, bucket_size=BUCKETS, max_position=MAX_POS, device=dev)
    rel_pos = build_relative_position(L, L, bucket_size=BUCKETS, max_position=MAX_POS, device=dev)

    def fused_step():
        out, _, _, _ = ops.attention(*leaves, table, None, None, A, scale)
        torch.autograd.grad(out, leaves, dout)

    def eager_step():
        out, _ = unfused_attention(*leaves, rel_pos, None, A, scale, ["c2p", "p2c"])
        torch.autograd.grad(out, leaves, dout)

    def timed(fn, warm, n):
        for _ in range(warm):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    f = 3 * flops_fwd(B, L, H, D, R)
    res = {"workload": "eager", "description": desc, "dtype": "fp32" if args.fp32 else "bf16"}
    # warm-up long enough (over 0.1 s) for the clocks to settle under either
    for name, fn, warm, n in (("fused", fused_step, 300, 50), ("eager_torch_ops", eager_step, 10, 20)):
        ms = timed(fn, warm, n)
        res[name + "_ms"] = round(ms, 4)
        res[name + "_tflops"] = round(f / (ms * 1e-3) / 1e12, 1)
    res["speedup"] = round(res["eager_torch_ops_ms"] / res["fused_ms"], 2)
    res["eager_peak_mem_gib"] = round(torch.cuda.max_memory_allocated(dev) / 2**30, 1)
    print(json.dumps(res), flush=True)


def run_compiled_layer(args) -> None:
    """C5 as BASELINE states it: one DeBERTa-v3-large-shaped attention
    layer (hidden 1024, 16 heads x 64, relative projections shared with the
    keys, c2p|p2c, full mask) fwd+bwd in bf16 inside torch.compile
    (inductor), so the op runs through its fake implementations.  Prints the
    step time and TFLOP/s of the op's algorithmic count; the projections
    (four 1024 x 1024 Linear layers on 32768 tokens, and the two on the
    relative table) run in hipBLASLt inside the same step."""
    import torch

    import deberta_amd

    dev = torch.device("cuda:0")
    Bc, Lc, Hc, hid = 64, 512, 16, 1024
    cfg = type("Cfg", (), dict(hidden_size=hid, num_attention_heads=Hc, share_att_key=True,
                               pos_att_type="p2c|c2p", relative_attention=True, position_buckets=BUCKETS,
                               max_relative_positions=-1, max_position_embeddings=MAX_POS,
                               hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0))()
    torch.manual_seed(0)
    layer = deberta_amd.DisentangledSelfAttention(cfg).to(dev, torch.bfloat16)
    for prm in layer.parameters():
        torch.nn.init.normal_(prm, 0.0, 0.02) if prm.dim() > 1 else torch.nn.init.zeros_(prm)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(Bc, Lc, hid, generator=g).to(dev, torch.bfloat16).requires_grad_(True)
    rel = (torch.randn(2 * BUCKETS, hid, generator=g) * 0.02).to(dev, torch.bfloat16).requires_grad_(True)
    dout = torch.randn(Bc, Lc, hid, generator=g).to(dev, torch.bfloat16)
    rel_pos = deberta_amd.build_relative_position(Lc, Lc, bucket_size=BUCKETS, max_position=MAX_POS, device=dev)
    compiled = torch.compile(layer)

    def step():
        out, _ = compiled(x, None, relative_pos=rel_pos, rel_embeddings=rel)
        out.backward(dout)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    n = max(3, args.steps)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n
    f_op = 3 * flops_fwd(Bc, Lc, Hc, D, R)
    f_proj = 3 * (2.0 * 3 * Bc * Lc * hid * hid + 2.0 * 2 * (2 * BUCKETS) * hid * hid)
    print(
        json.dumps(
            {
                "workload": "C5layer",
                "description": WORKLOADS["C5layer"][4],
                "ms_per_step": round(ms, 4),
                "tflops_op_count": round(f_op / (ms * 1e-3) / 1e12, 2),
                "tflops_with_projections": round((f_op + f_proj) / (ms * 1e-3) / 1e12, 2),
                "steps": n,
                "data": "synthetic hidden states, random init",
            }
        ),
        flush=True,
    )


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(c2_runs: int = 3, slice_budget_s: float = 5.0) -> dict:
    """fp32 eager oracle fwd+bwd (the reference's op chain restated) on the
    host's cores at the headline shape, B=32 whole: one warm-up step, then
    the median of c2_runs timed steps (BASELINE configs[1] as its CPU
    figure is specified).  Also reported: the rate over about slice_budget_s
    seconds of 2-row slices of the same shape, whose tensors fit the host's
    caches (several times the whole batch's rate: a slice rate is no
    estimate of the full step)."""
    import torch

    from oracle import eager

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rel = eager.relative_positions(L, L, BUCKETS, MAX_POS)

    def make(b):
        g = torch.Generator().manual_seed(0)
        q, k, v = (torch.randn(b, H, L, D, generator=g, requires_grad=True) for _ in range(3))
        kr, qr = (torch.randn(H, R, D, generator=g, requires_grad=True) for _ in range(2))
        dout = torch.randn(b, H, L, D, generator=g)

        def step():
            ctx, _ = eager.attend(q, k, v, kr, qr, rel, None, types=["c2p", "p2c"], att_span=A)
            torch.autograd.grad(ctx, (q, k, v, kr, qr), dout)

        return step

    step = make(B)
    t0 = time.perf_counter()
    step()  # warm-up
    warm = time.perf_counter() - t0
    ts = []
    for _ in range(c2_runs):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    del step
    med = sorted(ts)[len(ts) // 2]
    f_step = 3 * flops_fwd(B, L, H, D, R)

    b = 2
    step = make(b)
    step()  # warm-up
    runs = 0
    t0 = time.perf_counter()
    while True:
        step()
        runs += 1
        total = time.perf_counter() - t0
        if total >= slice_budget_s:
            break
    c1 = c1_cpu_forward()
    return {
        "value": round(f_step / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"fp32 eager oracle fwd+bwd at the headline shape B={B} L={L} H={H} D={D} R={R} (no mask): "
        f"median of {c2_runs} steps after one warm-up step ({warm:.1f} s): "
        + ", ".join(f"{t:.2f}" for t in ts)
        + f" s; CPU: {cpu_model()}",
        "ms_per_step": round(med * 1e3, 1),
        "slices": {
            "tflops": round(runs * 3 * flops_fwd(b, L, H, D, R) / total / 1e12, 4),
            "sample": f"{runs} runs of {b} batch rows of the same shape in {total:.1f} s "
            f"({total / runs * 1e3:.1f} ms per run)",
        },
        "c1_forward": c1,
    }


def c1_cpu_forward(runs: int = 20) -> dict:
    """BASELINE configs[0] on the host: the oracle's restatement of the
    reference module, forward only, fp32, B=2, L=128, hidden 128, 4 heads x
    32, buckets 256, max relative positions 512, relative embeddings
    [512, 128]; hidden states N(0, 1), weights N(0, 0.02) from seed 0,
    all-ones mask.  Median wall time over `runs` forwards."""
    import torch

    from oracle import eager

    cfg = eager.make_config(hidden_size=128, num_attention_heads=4, position_buckets=256, max_relative_positions=512)
    torch.manual_seed(0)
    m = eager.EagerDisentangledSelfAttention(cfg).eval()
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        for n_, p_ in m.named_parameters():
            p_.copy_(torch.randn(p_.shape, generator=g) * 0.02 if n_.endswith("weight") else torch.zeros_like(p_))
    x = torch.randn(2, 128, 128, generator=g)
    rel = torch.randn(512, 128, generator=g) * 0.02
    mask = torch.ones(2, 1, 1, 128, dtype=torch.bool)
    ts = []
    with torch.no_grad():
        m(x, mask, rel_embeddings=rel)
        for _ in range(runs):
            t0 = time.perf_counter()
            m(x, mask, rel_embeddings=rel)
            ts.append(time.perf_counter() - t0)
    ms = sorted(ts)[len(ts) // 2] * 1e3
    f = flops_fwd(2, 128, 4, 32, 512)
    return {"ms": round(ms, 3), "gflops": round(f / (ms * 1e-3) / 1e9, 2), "flop": f,
            "sample": "BASELINE configs[0]: oracle module forward, fp32, B=2 L=128 H=4 D=32, median of 20"}


def masked_figures(dev, names=("C2pad", "C4seg"), warmup: int = 100, steps: int = 20) -> dict:
    """Step time of the masked BASELINE workloads, for the record of the
    default run (reference figures, not the metric): each workload's inputs
    and mask are drawn as `--workload NAME` draws them (so the figures agree
    with those runs), then `warmup` untimed and `steps` timed fwd+bwd steps
    of the op between two HIP events.  TFLOP/s are counted over kept pairs
    and live rows."""
    import torch

    from deberta_amd import ops
    from deberta_amd.masks import kernel_masks
    from deberta_amd.relpos import relative_offset_table

    res = {}
    for name in names:
        b, l, h, kind, _ = WORKLOADS[name]
        g = torch.Generator(device="cpu").manual_seed(0)
        mk = lambda *s: torch.randn(*s, generator=g).to(device=dev, dtype=torch.bfloat16)
        q, k, v = mk(b, l, h, D), mk(b, l, h, D), mk(b, l, h, D)
        kr, qr = mk(h, R, D), mk(h, R, D)
        dout = mk(b, l, h, D)
        leaves = (q, k, v, kr, qr)
        for t in leaves:
            t.requires_grad_(True)
        table = relative_offset_table(l, l, bucket_size=BUCKETS, max_position=MAX_POS, device=dev)
        scale = 1.0 / math.sqrt(D * 3)
        mask, kept_pairs, live_rows = workload_mask(kind, b, l, g, dev)
        kk, pk = kernel_masks(mask, b, l, l, dev)

        def step():
            out, _, _, _ = ops.attention(q, k, v, kr, qr, table, kk, pk, A, scale, True, None, 0, None)
            return torch.autograd.grad(out, leaves, dout)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        sp = torch.cuda.current_stream(dev).cuda_stream
        ev = HipEvents(2)
        ev.record(0, sp)
        for _ in range(steps):
            step()
        ev.record(1, sp)
        torch.cuda.synchronize()
        ms = ev.ms(0, 1) / steps
        f_kept = 3.0 * h * D * (4.0 * kept_pairs + 4.0 * R * live_rows)
        res[name] = {
            "ms_per_step": round(ms, 4),
            "tflops_kept_pairs": round(f_kept / (ms * 1e-3) / 1e12, 2),
            "kept_pair_fraction": round(kept_pairs / (b * l * l), 4),
            "steps": steps,
            "warmup": warmup,
        }
        del q, k, v, kr, qr, dout, mask, kk, pk, leaves
    return res


def cpu_c4(q, k, v, kr, qr, dout, mask, table_l: int, f_dense: float, f_kept: float) -> dict:
    """BASELINE configs[3] on the host: one fp32 eager-oracle fwd+bwd (no
    warm-up: its (4, 12, 4096, 4096) fp32 tensors take about 18 GB) on the
    workload's own inputs and dense document mask, all host cores."""
    import torch

    from oracle import eager

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    to_cpu = lambda t: t.detach().float().cpu()
    heads = lambda t: to_cpu(t).permute(0, 2, 1, 3).contiguous().requires_grad_(True)
    qc, kc, vc = heads(q), heads(k), heads(v)
    krc, qrc = (to_cpu(t).requires_grad_(True) for t in (kr, qr))
    doc = to_cpu(dout).permute(0, 2, 1, 3).contiguous()
    keep = mask.cpu()
    rel = eager.relative_positions(table_l, table_l, BUCKETS, MAX_POS)
    t0 = time.perf_counter()
    ctx, _ = eager.attend(qc, kc, vc, krc, qrc, rel, keep, types=["c2p", "p2c"], att_span=A)
    torch.autograd.grad(ctx, (qc, kc, vc, krc, qrc), doc)
    sec = time.perf_counter() - t0
    return {
        "s_per_step": round(sec, 2),
        "tflops_dense_count": round(f_dense / sec / 1e12, 4),
        "tflops_kept_pairs": round(f_kept / sec / 1e12, 4),
        "cores": cores,
        "kind": "port",
        "sample": f"fp32 eager oracle fwd+bwd, one step (no warm-up), B={qc.shape[0]} L={table_l} H={qc.shape[1]} "
        f"D={qc.shape[3]} with the dense document mask; CPU: {cpu_model()}",
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # The GPU's clocks need about 60 to 80 steps (some 30 ms) of sustained
    # load to settle: at B=32, L=512 the step takes 0.52 ms over the first 20
    # steps of a process, 0.44 ms from the 80th on, and ramps again after an
    # idle second.  The per-kernel timing runs before the timed steps and
    # covers the ramp; the warm-up steps follow it.
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument(
        "--no-masked",
        action="store_true",
        help="skip the short C2pad / C4seg step timings that follow the headline's timed steps",
    )
    ap.add_argument(
        "--workload",
        choices=sorted(WORKLOADS),
        default="headline",
        help="shape and mask; the headline is the metric, the others print reference figures",
    )
    ap.add_argument(
        "--dropout",
        type=float,
        default=0.0,
        help="attention dropout probability in the kernels (a fresh seed per step); reference figures, not the metric",
    )
    ap.add_argument(
        "--kernels-only",
        action="store_true",
        help="only run each kernel --steps times (for rocprofv3 counter passes); prints per-kernel times",
    )
    ap.add_argument(
        "--atomics-probe",
        action="store_true",
        help="only time the fp32 atomic flush a backward without dS would make at the workload's shape, and exit",
    )
    ap.add_argument(
        "--fp32",
        action="store_true",
        help="with --workload eager: both sides in float32 (the reference's train.mixed_precision=no)",
    )
    ap.add_argument(
        "--cpu-c4",
        action="store_true",
        help="with --workload C4: also time one fp32 oracle fwd+bwd of the same step on the host (about 18 GB)",
    )
    ap.add_argument(
        "--copy-probe-mib",
        type=int,
        default=0,
        help="also run a plain device copy of this many MiB (calibrates FETCH_SIZE / WRITE_SIZE)",
    )
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: the op has no cross-GPU exchange and this build runs on a "
            f"single MI355X (asked for --gpus {args.gpus}).",
            file=sys.stderr,
        )
        sys.exit(2)

    if args.workload == "C3":
        run_encoder(args)
        return
    if args.workload == "C5layer":
        run_compiled_layer(args)
        return
    if args.workload == "plain":
        run_plain(args)
        return
    if args.workload == "eager":
        run_eager(args)
        return

    import torch

    import deberta_amd  # noqa: F401
    from deberta_amd import _lib, ops
    from deberta_amd.masks import kernel_masks
    from deberta_amd.relpos import relative_offset_table

    lib = _lib.load()
    dev = torch.device("cuda:0")
    B, L, H, mask_kind, wl_desc = WORKLOADS[args.workload]
    if args.atomics_probe:
        print(json.dumps({"dsfree_flush_probe": dsfree_flush_probe(dev, B, H, L)}), flush=True)
        return
    headline = args.workload == "headline" and not args.dropout
    drop_t = ops.dropout_threshold(args.dropout) if args.dropout > 0 else 0
    if args.dropout > 0 and not 0 < drop_t < 65536:
        sys.exit(f"--dropout {args.dropout} has no kernel form")
    g = torch.Generator(device="cpu").manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=g).to(device=dev, dtype=torch.bfloat16)
    q, k, v = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, R, D), mk(H, R, D)
    dout = mk(B, L, H, D)
    for t in (q, k, v, kr, qr):
        t.requires_grad_(True)
    table = relative_offset_table(L, L, bucket_size=BUCKETS, max_position=MAX_POS, device=dev)
    scale = 1.0 / math.sqrt(D * 3)
    leaves = (q, k, v, kr, qr)
    mask, kept_pairs, live_rows = workload_mask(mask_kind, B, L, g, dev)
    kk, pk = kernel_masks(mask, B, L, L, dev)

    def step():
        seed = ops.draw_dropout_seed() if drop_t else None
        out, _, _, _ = ops.attention(q, k, v, kr, qr, table, kk, pk, A, scale, True, None, drop_t, seed)
        return torch.autograd.grad(out, leaves, dout)

    if args.copy_probe_mib:
        n = args.copy_probe_mib * (1 << 20) // 4
        src_t = torch.ones(n, dtype=torch.float32, device=dev)
        dst_t = torch.empty_like(src_t)
        for _ in range(3):
            dst_t.copy_(src_t)
        torch.cuda.synchronize()
        del src_t, dst_t

    if args.kernels_only:
        # the same sustained load before the per-kernel timing as in a full
        # run (the GPU's clocks settle under it)
        for _ in range(args.warmup + args.steps):
            step()
        torch.cuda.synchronize()

    f_fwd = flops_fwd(B, L, H, D, R)
    f_step = 3 * f_fwd
    # masked work counted over kept pairs and live rows only (the skipped
    # pairs are not work): 3 x (4 H D kept + 4 H D R live)
    f_kept = 3.0 * H * D * (4.0 * kept_pairs + 4.0 * R * live_rows)

    # ---- per-kernel times: each launch timed on the stream it runs on ------------
    stream = torch.cuda.current_stream(dev)
    dseed = ops.draw_dropout_seed() if drop_t else None
    out, lse, bias, dbits = torch.ops.deberta_amd.dsa_fwd(
        q, k, v, kr, qr, table, kk, pk, A, scale, True, None, drop_t, dseed
    )
    f32 = dict(dtype=torch.float32, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dkr, dqr = torch.zeros((H, R, D), **f32), torch.zeros((H, R, D), **f32)
    bargs = ops.fill_bwd_args(
        dout, q, k, v, kr, qr, table, kk, pk, out, lse, bias, A, scale, dq, dk, dv, dkr, dqr,
        dropout_t=drop_t, dropout_seed=dseed, dropout_bits=dbits,
    )
    ws = torch.empty((ops.bwd_workspace_bytes(bargs),), dtype=torch.uint8, device=dev)
    bargs.workspace, bargs.workspace_bytes = ws.data_ptr(), ws.numel()
    fargs = bargs.fwd
    # launch-order scratch under masks, table copies, dropout's keep bits
    nfws = lib.dsa_fwd_workspace_bytes(ctypes.byref(fargs))
    fws = torch.empty((max(nfws, 16),), dtype=torch.uint8, device=dev)
    if nfws:
        fargs.workspace, fargs.workspace_bytes = fws.data_ptr(), nfws
    sptr = ctypes.c_void_p(stream.cuda_stream)

    def run_fwd():
        _lib.check(lib.dsa_fwd(ctypes.byref(fargs), sptr), "dsa_fwd")

    def run_stage(st):
        def f():
            bargs.stages = st
            _lib.check(lib.dsa_bwd(ctypes.byref(bargs), sptr), "dsa_bwd")

        return f

    bh = B * H * D
    f_dkdv = bh * (6.0 * L * L + 2.0 * L * R)
    f_dq = bh * (2.0 * L * L + 2.0 * L * R)
    f_table = bh * 4.0 * L * R
    # Per-kernel times in settled steps: K more fwd+bwd steps through the C
    # ABI, one call per stage with a HIP event between calls on the launch
    # stream.  The kernels and their order are the op's (DQ with TABLE is its
    # one fused launch), so each entry is that kernel's duration inside a
    # step at the clocks of a sustained run; the forward's entry includes its
    # table copy (dsa_table_ks_kernel), which the same call launches first.
    staged = [
        ("dsa_fwd_kernel (after dsa_table_ks_kernel" + (" and dsa_dropout_bits_kernel)" if drop_t else ")"), run_fwd,
         f_fwd),
        ("dsa_bwd_prep_kernel", run_stage(_lib.DSA_STAGE_PREP), 0.0),
        ("dsa_bwd_dkdv_kernel", run_stage(_lib.DSA_STAGE_DKDV), f_dkdv),
        ("dsa_bwd_dqtab_kernel", run_stage(_lib.DSA_STAGE_DQ | _lib.DSA_STAGE_TABLE), f_dq + f_table),
        ("dsa_bwd_fold_kernel", run_stage(_lib.DSA_STAGE_SUM), 0.0),
    ]
    n_k = args.steps if args.kernels_only else max(10, args.steps)
    # Sustained load before the per-kernel timing: 300 stage-split steps
    # (about 0.13 s) bring the clocks of a fresh process to their settled
    # level (100 were not always enough on a box's first run); with
    # --kernels-only the op's steps above already did.
    for _ in range(20 if args.kernels_only else 300):
        for _, fn, _ in staged:
            fn()
    ns_ = len(staged) + 1
    evk = HipEvents(n_k * ns_)
    for n_ in range(n_k):
        evk.record(n_ * ns_, stream.cuda_stream)
        for i_, (_, fn, _) in enumerate(staged):
            fn()
            evk.record(n_ * ns_ + i_ + 1, stream.cuda_stream)
    torch.cuda.synchronize()
    per_kernel = {}
    for i_, (name, _, fl) in enumerate(staged):
        ms = sum(evk.ms(n_ * ns_ + i_, n_ * ns_ + i_ + 1) for n_ in range(n_k)) / n_k
        per_kernel[name] = {"ms": round(ms, 5), "tflops": round(fl / (ms * 1e-3) / 1e12, 2) if fl else None}
    flops_of = {name: fl for name, _, fl in staged}
    # the dq and table kernels launched apart (each alone, back to back):
    # reference figures for the two parts of the fused launch
    alone = {
        "dsa_bwd_dq_kernel": (run_stage(_lib.DSA_STAGE_DQ), f_dq),
        "dsa_bwd_table_kernel": (run_stage(_lib.DSA_STAGE_TABLE), f_table),
    }
    per_kernel_alone = {}
    for name, (fn, fl) in alone.items():
        for _ in range(3):
            fn()
        a_, b_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a_.record(stream)
        for _ in range(n_k):
            fn()
        b_.record(stream)
        torch.cuda.synchronize()
        ms = a_.elapsed_time(b_) / n_k
        per_kernel_alone[name] = {"ms": round(ms, 5), "tflops": round(fl / (ms * 1e-3) / 1e12, 2)}
    dom = max((n for n in per_kernel if flops_of[n] > 0), key=lambda n: per_kernel[n]["ms"])
    dom_ms = per_kernel[dom]["ms"]
    achieved = flops_of[dom] / (dom_ms * 1e-3) / 1e12
    if args.kernels_only:
        print(json.dumps({"per_kernel": per_kernel, "per_kernel_alone": per_kernel_alone}), flush=True)
        return
    # The stage calls' buffers go back to the caching allocator, which hands
    # the same blocks to the op's steps below (same sizes).
    del out, lse, bias, dbits, dq, dk, dv, dkr, dqr, bargs, fargs, ws, fws
    torch.cuda.synchronize()

    # ---- the timed steps ----------------------------------------------------------
    # They run after the per-kernel timing above, whose stage calls keep the
    # GPU under sustained load for about 30 ms: its clocks take some 80 steps
    # to settle after a process starts (0.52 ms a step over the first 20, 0.44
    # from the 80th on), so the W warm-up steps alone would time the ramp when
    # W is small.  The op's own first steps after the stage calls still ran
    # slower (with the driver's --warmup 5, the K = 20 steps after them
    # averaged 0.443 ms against 0.427 for the next 20 on one box), so
    # SETTLE_STEPS untimed steps of the op come first, whatever W is: then W
    # untimed warm-up steps and exactly K timed fwd+bwd steps of the op.
    ms_step = wall = ms_median = ms_p10 = ms_p90 = float("nan")
    for _ in range(SETTLE_STEPS + args.warmup):
        step()
    torch.cuda.synchronize()
    sp = torch.cuda.current_stream(dev).cuda_stream
    # The timed region: exactly K steps between two events (an event between
    # steps is itself a few microseconds of queue work: 4.4 us a step in a
    # kernel trace, the only gap between the step's kernels).
    t0 = time.perf_counter()
    ev2 = HipEvents(2)
    ev2.record(0, sp)
    for _ in range(args.steps):
        step()
    ev2.record(1, sp)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = ev2.ms(0, 1) / args.steps
    # Then K more steps with an event between consecutive ones: per-step
    # times for the median and p10 / p90.
    evs = HipEvents(args.steps + 1)
    evs.record(0, sp)
    for n_ in range(args.steps):
        step()
        evs.record(n_ + 1, sp)
    torch.cuda.synchronize()
    per_step = sorted(evs.ms(n_, n_ + 1) for n_ in range(args.steps))
    pct = lambda f: per_step[min(len(per_step) - 1, int(round(f * (len(per_step) - 1))))]
    ms_median, ms_p10, ms_p90 = pct(0.5), pct(0.1), pct(0.9)
    tflops = f_step / (ms_step * 1e-3) / 1e12
    if not headline:
        # reference figures of another shape: not the metric (no roofline or
        # CPU leg; per-kernel TFLOP/s use the dense counts)
        print(
            json.dumps(
                {
                    "workload": args.workload,
                    "description": wl_desc,
                    "attention_dropout": args.dropout,
                    "ms_per_step": round(ms_step, 4),
                    "tflops_dense_count": round(tflops, 2),
                    "kept_pair_fraction": round(kept_pairs / (B * L * L), 4),
                    "tflops_kept_pairs": round(f_kept / (ms_step * 1e-3) / 1e12, 2),
                    "steps": args.steps,
                    "per_kernel": per_kernel,
                    "per_kernel_alone": per_kernel_alone,
                    **(
                        {"cpu_c4": cpu_c4(q, k, v, kr, qr, dout, mask, L, f_step, f_kept)}
                        if args.cpu_c4 and args.workload == "C4"
                        else {}
                    ),
                }
            ),
            flush=True,
        )
        return

    res = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "fused disentangled attention fwd+bwd (c2p|p2c), BASELINE configs[1] shape, all-ones mask",
            "batch": B,
            "seq_len": L,
            "heads": H,
            "head_dim": D,
            "position_buckets": BUCKETS,
            "max_relative_positions": MAX_POS,
            "rel_rows": R,
            "flop_per_step": f_step,
        },
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "step_ms_median_p10_p90": [round(ms_median, 4), round(ms_p10, 4), round(ms_p90, 4)],
        "tflops_at_median_step": round(f_step / (ms_median * 1e-3) / 1e12, 2),
        "mfma_peak_measured": mfma_peak_probe(dev),
        "per_kernel": per_kernel,
        "per_kernel_alone": per_kernel_alone,
        "roofline": {
            "kernel": dom,
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": hbm_bytes(dom),
            "traffic_unit": "bytes/launch",
        },
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_masked:
        # after the headline's timed steps, so they cannot affect its figures;
        # an error here is reported in the line rather than losing the line
        try:
            res["masked_workloads"] = masked_figures(dev)
        except Exception as e:  # noqa: BLE001
            res["masked_workloads"] = {"error": f"{type(e).__name__}: {e}"}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
