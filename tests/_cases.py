"""Seeded inputs and the two sides of an op-level parity check: the HIP op
(through torch.ops.deberta_amd) and the CPU oracle (oracle.eager.attend +
autograd), on identical values."""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from oracle import eager


@dataclass
class Case:
    B: int
    H: int
    L: int
    D: int
    buckets: int = 256
    max_pos: int = 512
    types: str = "c2p|p2c"
    mask: str = "none"  # none | key | pair | pair_auto | seg | seg_mixed | dead
    seed: int = 0
    Lk: Optional[int] = None
    std: float = 1.0
    ramp: float = 0.0  # key j scaled by 1 + ramp * j / Lk (score maxima grow along the keys)
    dropout: float = 0.0  # attention dropout probability (kernel threshold round(p * 65536))
    drop_seed: int = 0x1234_5678_9ABC_DEF

    @property
    def drop_t(self) -> int:
        return int(round(self.dropout * 65536)) if self.dropout > 0 else 0

    @property
    def A(self) -> int:
        return self.buckets if self.buckets > 0 else self.max_pos

    @property
    def type_list(self) -> list[str]:
        return eager.pos_att_types(self.types)


def make_inputs(c: Case) -> dict:
    """fp32 CPU tensors drawn from one generator in a fixed order:
    q, k, v [B, L, H, D]; kr, qr [H, 2A, D]; dO [B, L, H, D]; mask."""
    g = torch.Generator().manual_seed(c.seed)
    Lk = c.Lk or c.L
    q = torch.randn(c.B, c.L, c.H, c.D, generator=g) * c.std
    k = torch.randn(c.B, Lk, c.H, c.D, generator=g) * c.std
    v = torch.randn(c.B, Lk, c.H, c.D, generator=g)
    kr = torch.randn(c.H, 2 * c.A, c.D, generator=g) * c.std
    qr = torch.randn(c.H, 2 * c.A, c.D, generator=g) * c.std
    dout = torch.randn(c.B, c.L, c.H, c.D, generator=g)
    if c.ramp:
        k = k * (1 + c.ramp * torch.arange(Lk, dtype=torch.float32) / Lk)[None, :, None, None]
    mask = seg = None
    if c.mask == "key":
        lens = torch.randint(max(1, c.L // 8), c.L + 1, (c.B,), generator=g)
        lens[0] = c.L
        mask = (torch.arange(c.L)[None, :] < lens[:, None])[:, None, None, :]
    elif c.mask in ("pair", "pair_auto", "seg"):
        # packed documents: contiguous runs of ids 1, 2, ..., a padded tail (id 0)
        ids = torch.zeros(c.B, c.L, dtype=torch.long)
        for b in range(c.B):
            pos, doc = 0, 1
            while pos < c.L:
                n = int(torch.randint(1, max(2, c.L // 3), (1,), generator=g))
                ids[b, pos : pos + n] = doc
                pos += n
                doc += 1
            pad = int(torch.randint(0, c.L // 4 + 1, (1,), generator=g))
            if pad:
                ids[b, c.L - pad :] = 0
        mask = eager.doc_block_mask(ids)[:, None]
        if c.mask == "seg":
            seg = ids
    elif c.mask == "seg_mixed":
        # interleaved segments (ids repeat out of order) and scattered
        # inactive tokens: every tile's segment range overlaps
        ids = (torch.arange(c.L)[None, :] // 7 + torch.arange(c.B)[:, None]) % 3 + 1
        ids = ids * (torch.rand(c.B, c.L, generator=g) > 0.1)
        mask = eager.doc_block_mask(ids)[:, None]
        seg = ids
    elif c.mask == "dead":
        keep = torch.rand(c.B, c.L, c.L, generator=g) < 0.5
        live = torch.rand(c.B, c.L, generator=g) < 0.7
        eye = torch.eye(c.L, dtype=torch.bool)
        keep = (keep & ~eye) | (eye & live[:, :, None])
        mask = keep[:, None]
    return dict(q=q, k=k, v=v, kr=kr, qr=qr, dout=dout, mask=mask, seg=seg)


def oracle_run(c: Case, x: dict, dtype: torch.dtype, grads: bool = True) -> dict:
    """Oracle forward (+ autograd backward) in fp32 on the values the kernel
    sees (inputs rounded to `dtype` first)."""
    types = c.type_list
    r = lambda t: t.to(dtype).to(torch.float32).detach().clone().requires_grad_(grads)
    q, k, v = (r(x[n]).permute(0, 2, 1, 3) for n in ("q", "k", "v"))
    kr = r(x["kr"]) if ("c2p" in types or "p2p" in types) else None
    qr = r(x["qr"]) if ("p2c" in types or "p2p" in types) else None
    use_rel = kr is not None or qr is not None
    Lk = c.Lk or c.L
    rel = eager.relative_positions(c.L, Lk, c.buckets, c.max_pos) if use_rel else None
    keep, p = None, 0.0
    if c.drop_t:
        from oracle.dropout import keep_mask

        keep = torch.from_numpy(keep_mask(c.drop_seed, c.drop_t, c.B, c.H, c.L, Lk))
        p = c.drop_t / 65536
    ctx, _ = eager.attend(
        q, k, v, kr, qr, rel, x["mask"], types=types, att_span=c.A, use_relative=use_rel, dropout_keep=keep,
        dropout_p=p,
    )
    out = ctx.permute(0, 2, 1, 3)
    res = {"out": out.detach()}
    if grads:
        dout = x["dout"].to(dtype).to(torch.float32)
        leaves = [t for t in (q, k, v, kr, qr) if t is not None]
        gs = torch.autograd.grad(out, leaves, dout, allow_unused=True)
        names = ["q", "k", "v"] + (["kr"] if kr is not None else []) + (["qr"] if qr is not None else [])
        for n, gval in zip(names, gs):
            gval = torch.zeros_like(leaves[names.index(n)]) if gval is None else gval
            res["d" + n] = gval.permute(0, 2, 1, 3).detach() if n in ("q", "k", "v") else gval.detach()
    return res


def hip_run(c: Case, x: dict, dtype: torch.dtype, device, grads: bool = True) -> dict:
    """The HIP op through the custom-op boundary (autograd for the backward)."""
    from deberta_amd import ops  # noqa: F401
    from deberta_amd.attention import relative_operands
    from deberta_amd.masks import kernel_masks
    from deberta_amd.relpos import relative_offset_table

    types = c.type_list
    Lk = c.Lk or c.L
    dev = lambda t: t.to(device=device, dtype=dtype).detach().clone().requires_grad_(grads)
    q, k, v = dev(x["q"]), dev(x["k"]), dev(x["v"])
    kr = dev(x["kr"]) if ("c2p" in types or "p2p" in types) else None
    qr = dev(x["qr"]) if ("p2c" in types or "p2p" in types) else None
    # p2p rides on the c2p term's query rows qc (autograd takes qc's
    # gradient back to q and qr)
    kr_op, qr_op, qc = relative_operands(types, q, kr, qr, c.A)
    table = None
    if kr is not None or qr is not None:
        table = relative_offset_table(c.L, Lk, bucket_size=c.buckets, max_position=c.max_pos, device=device)
    if x.get("seg") is not None:
        from deberta_amd.masks import SegmentMask

        mask = SegmentMask(x["seg"])
    else:
        mask = x["mask"].to(device) if x["mask"] is not None else None
    # "pair" keeps the dense document mask on the pair-mask kernels;
    # "pair_auto" lets kernel_masks turn it into segment ids
    kk, pk = kernel_masks(mask, c.B, c.L, Lk, device, segments_from_dense=c.mask != "pair")
    if c.mask == "pair_auto":
        assert pk is None and kk is not None and kk.dtype == torch.int32, "document mask not recognised"
    sf = 1 + sum(t in types for t in ("c2p", "p2c", "p2p"))
    scale = 1.0 / math.sqrt(c.D * sf)
    seed = torch.tensor([c.drop_seed], dtype=torch.int64) if c.drop_t else None
    out, lse, _, _ = torch.ops.deberta_amd.dsa_fwd(q, k, v, kr_op, qr_op, table, kk, pk, c.A, scale, True, qc, c.drop_t, seed)
    res = {"out": out.detach().float().cpu(), "lse": lse.detach().cpu()}
    if grads:
        dout = x["dout"].to(device=device, dtype=dtype)
        leaves = [t for t in (q, k, v, kr, qr) if t is not None]
        names = ["q", "k", "v"] + (["kr"] if kr is not None else []) + (["qr"] if qr is not None else [])
        gs = torch.autograd.grad(out, leaves, dout)
        for n, gval in zip(names, gs):
            res["d" + n] = gval.detach().float().cpu()
    torch.cuda.synchronize(device)
    return res


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float() - b.float()).abs().max()) if a.numel() else 0.0


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b|: the fp32 parity metric (relative to the
    tensor's scale, so near-zero entries do not dominate)."""
    if not b.numel():
        return 0.0
    den = float(b.float().abs().max())
    return max_abs(a, b) / max(den, 1e-30)
