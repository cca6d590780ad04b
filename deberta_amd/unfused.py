"""The attention in torch operations on the device, for the module cases the
fused kernels do not take.

``DisentangledSelfAttention.forward`` sends four cases here instead of to
``deberta_amd::dsa_fwd``:

* CPU tensors (the reference module is device-agnostic; the kernels run on
  the GPU only);
* ``output_attentions=True``: the probabilities are returned, so they are
  materialised;
* attention dropout in training mode with a probability the kernels
  cannot draw (below 2^-17 or above 1 - 2^-17; every other probability runs
  in the kernels): torch's dropout acts on the materialised probabilities;
* a ``relative_pos`` matrix that does not depend on ``i - j`` alone (the
  kernels take a per-offset table), used as given.

The function is the reference's score chain (deberta_v2_native.py:592-652
with the dynamic bias of :349-432 and the p2p term of :298-347): scores and
relative terms in float32, keep-mask fill with the float32 minimum, dead
query rows zeroed, softmax, dropout, then the value product.  It is written
on torch's device operations in this package (differentiable through
autograd) and is not the test oracle.  The value product runs in float32
(the reference multiplies in the value dtype): its result differs from the
reference's by the rounding of the probabilities to bf16 only.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn


def _rows(t: torch.Tensor) -> torch.Tensor:
    """``[B, L, H, D]`` -> contiguous float32 ``[B, H, L, D]``."""
    return t.float().permute(0, 2, 1, 3).contiguous()


def relative_terms(
    qh: torch.Tensor,
    kh: torch.Tensor,
    kr: Optional[torch.Tensor],
    qr: Optional[torch.Tensor],
    rel_pos: Optional[torch.Tensor],
    att_span: int,
    scale: float,
    types: list[str],
) -> Optional[torch.Tensor]:
    """The relative score term ``scale * (c2p + p2c + p2p)`` of float32
    ``[B, H, L, D]`` query and key rows as float32 ``(B, H, Lq, Lk)``, None
    when ``types`` names no relative term (deberta_v2_native.py:349-432 with
    the p2p term of :298-347; the terms are summed before they reach the
    scores, as the reference's bias is).  ``rel_pos``: the ``(Lq, Lk)``
    relative positions (bucketed, not clamped)."""
    if not any(t in types for t in ("c2p", "p2c", "p2p")):
        return None
    if rel_pos is None:
        raise ValueError("relative positions are required with c2p / p2c / p2p")
    Lq, Lk = qh.shape[2], kh.shape[2]
    A = int(att_span)
    rp = rel_pos.to(device=qh.device, dtype=torch.long).clamp(-A, A)
    fwd_idx = (rp + A).clamp(0, 2 * A - 1)  # (Lq, Lk): c2p and p2p rows
    total = None
    if "c2p" in types:
        if kr is None:
            raise RuntimeError("p2p/c2p path requires pos_key projection.")
        krt = kr.float().transpose(-1, -2).contiguous()  # (H, D, 2A)
        c2p = torch.matmul(qh, krt)  # (B, H, Lq, 2A)
        total = c2p.gather(-1, fwd_idx.expand(*c2p.shape[:2], Lq, Lk)) * scale
    if "p2c" in types:
        if qr is None:
            raise RuntimeError("p2p/p2c path requires pos_query projection.")
        qrt = qr.float().transpose(-1, -2).contiguous()
        p2c = torch.matmul(kh, qrt)  # (B, H, Lk, 2A)
        bwd_idx = (A - rp.t()).clamp(0, 2 * A - 1)  # (Lk, Lq)
        term = p2c.gather(-1, bwd_idx.expand(*p2c.shape[:2], Lk, Lq)).transpose(-1, -2) * scale
        total = term if total is None else total + term
    if "p2p" in types:
        if kr is None or qr is None:
            raise RuntimeError("p2p path requires both pos_key and pos_query projections.")
        # position-to-position: the positive half of the pos-query table,
        # row min(i, A - 1), against Kr at the c2p row
        pq = qr.float()[:, A:, :]  # (H, A, D)
        table = torch.matmul(pq, kr.float().transpose(-1, -2).contiguous())  # (H, A, 2A)
        rows = torch.arange(Lq, device=qh.device).clamp(max=A - 1)
        per_query = table.index_select(1, rows)  # (H, Lq, 2A)
        term = per_query.gather(-1, fwd_idx.expand(per_query.shape[0], Lq, Lk)) * scale
        term = term.unsqueeze(0).expand(qh.shape[0], -1, -1, -1)
        total = term if total is None else total + term
    return total


def unfused_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kr: Optional[torch.Tensor],
    qr: Optional[torch.Tensor],
    rel_pos: Optional[torch.Tensor],
    keep_mask: Optional[torch.Tensor],
    att_span: int,
    scale: float,
    types: list[str],
    dropout: Optional[nn.Module] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(context ``[B, Lq, H, D]`` in v's dtype, probabilities ``(B, H, Lq, Lk)``
    float32).

    q, k, v: ``[B, L, H, D]`` layers.  kr / qr: the projected relative tables
    ``(H, 2A, D)`` (None where no term needs them).  rel_pos: the ``(Lq, Lk)``
    relative positions (bucketed, not clamped), required with a relative
    term.  keep_mask: a bool keep mask broadcastable to ``(B, H, Lq, Lk)``
    (rank 4) or None.  types: the normalised ``pos_att_type``; scale = 1 /
    sqrt(D * scale_factor).  dropout: applied to the probabilities (as the
    module's ``dropout``)."""
    qh, kh, vh = _rows(q), _rows(k), _rows(v)
    scores = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) * scale
    rel = relative_terms(qh, kh, kr, qr, rel_pos, att_span, scale, types)
    if rel is not None:
        scores = scores + rel
    live = None
    if keep_mask is not None:
        scores = scores.masked_fill(~keep_mask, torch.finfo(scores.dtype).min)
        if keep_mask.shape[-2] == 1:
            live = keep_mask.transpose(-2, -1)
        else:
            live = torch.diagonal(keep_mask, dim1=-2, dim2=-1).unsqueeze(-1)
        scores = torch.where(live, scores, torch.zeros_like(scores))
    probs = torch.softmax(scores, dim=-1)
    if dropout is not None:
        probs = dropout(probs)
    if live is not None:
        probs = probs * live.to(probs.dtype)
    ctx = torch.matmul(probs, vh)  # (B, H, Lq, D)
    return ctx.permute(0, 2, 1, 3).to(v.dtype), probs
