"""Eager torch-CPU restatement of the reference's disentangled attention.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Each function names the
reference lines it restates (pszemraj/deberta, paths relative to
src/deberta/).  Semantics, dtype handling and operation order follow the
reference so that fp32 results agree with it to rounding.
"""

from __future__ import annotations

import math
from types import SimpleNamespace
from typing import Any, Optional

import torch
import torch.nn as nn


# --- modeling/deberta_v2_native.py:28-48 -------------------------------------
def pos_att_types(raw: Any) -> list[str]:
    if raw is None:
        return []
    if isinstance(raw, str):
        parts = raw.replace(",", "|").split("|")
    elif isinstance(raw, (list, tuple, set)):
        parts = [str(x) for x in raw]
    else:
        parts = [str(raw)]
    return [p.strip().lower() for p in parts if p.strip()]


# --- modeling/deberta_v2_native.py:51-84 -------------------------------------
def log_bucket(rel: torch.Tensor, bucket_size: int, max_position: int) -> torch.Tensor:
    if int(max_position) > 0:
        rel = rel.clamp(min=1 - int(max_position), max=int(max_position) - 1)
    sgn = torch.sign(rel)
    mid = int(bucket_size) // 2
    if mid <= 1:
        return rel
    mag = rel.abs().clamp_min(1)
    base = math.log(max(float(max_position - 1), float(mid + 1)) / float(mid))
    if base <= 0.0:
        return rel
    far = torch.ceil(torch.log(mag.float() / float(mid)) / base * float(mid - 1)) + float(mid)
    out = torch.where(mag < mid, mag.to(far.dtype), far) * sgn.to(far.dtype)
    return out.to(torch.long)


# --- modeling/deberta_v2_native.py:87-112 ------------------------------------
def relative_positions(query_len: int, key_len: int, bucket_size: int, max_position: int) -> torch.Tensor:
    rel = torch.arange(query_len, dtype=torch.long)[:, None] - torch.arange(key_len, dtype=torch.long)[None, :]
    if int(bucket_size) > 0 and int(max_position) > 0:
        rel = log_bucket(rel, bucket_size, max_position)
    return rel.to(torch.long)


# --- modeling/mask_utils.py:8-32 ---------------------------------------------
def keep_mask(mask: Any, name: str = "attention_mask") -> torch.Tensor:
    if not isinstance(mask, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(mask)!r}.")
    if mask.dtype == torch.bool:
        return mask
    if torch.is_floating_point(mask):
        raise ValueError(f"{name} must be a bool/integer keep-mask tensor.")
    return mask != 0


# --- modeling/deberta_v2_native.py:1049-1068 ---------------------------------
def encoder_mask(mask: torch.Tensor) -> torch.Tensor:
    m = keep_mask(mask)
    if m.ndim <= 2:
        return m[:, None, None, :]
    if m.ndim == 3:
        return m[:, None]
    if m.ndim == 4:
        return m if m.shape[1] == 1 else m.any(dim=1, keepdim=True)
    raise ValueError(f"attention_mask must be rank-2/3/4; got rank={m.ndim}")


# --- training/compile.py:310-349 ----------------------------------------------
def doc_block_mask(doc_ids: torch.Tensor) -> torch.Tensor:
    if doc_ids.ndim != 2:
        raise ValueError("doc_ids must be rank-2 (B,S)")
    S = doc_ids.shape[1]
    diag = torch.eye(S, dtype=torch.bool)
    act = doc_ids != 0
    m = (doc_ids[:, :, None] == doc_ids[:, None, :]) & act[:, :, None] & act[:, None, :]
    cls = torch.zeros(S, dtype=torch.bool)
    cls[0] = True
    m = m | (~act[:, :, None] & cls[None, None, :])
    return (m & ~diag) | (diag & act[:, :, None])


# --- modeling/deberta_v2_native.py:235-271 ------------------------------------
def canonical_rel(rp: Optional[torch.Tensor], Lq: int, Lk: int, buckets: int, max_pos: int) -> torch.Tensor:
    if rp is None:
        return relative_positions(Lq, Lk, buckets, max_pos)
    rp = rp.long()
    if rp.ndim == 4:
        rp = rp[0, 0]
    elif rp.ndim == 3:
        rp = rp[0]
    elif rp.ndim != 2:
        raise ValueError(f"relative_pos must be rank-2/3/4, got rank={rp.ndim}")
    return rp[:Lq, :Lk]


# --- modeling/deberta_v2_native.py:298-347 (p2p), 349-432 (einsum variant),
#     434-528 (bmm variant) — on already projected tables --------------------
def relative_bias(
    q: torch.Tensor,
    k: torch.Tensor,
    kr: Optional[torch.Tensor],
    qr: Optional[torch.Tensor],
    rel: torch.Tensor,
    att_span: int,
    types: list[str],
    scale_factor: int,
    head_dim: int,
    variant: str = "einsum",
) -> torch.Tensor:
    """c2p + p2c (+ p2p) bias ``(B, H, Q, K)``; q, k are ``(B, H, L, D)``,
    kr/qr ``(H, 2A, D)`` already in q's dtype."""
    B, H, Lq, _ = q.shape
    Lk = k.shape[2]
    A = int(att_span)
    rel = rel.clamp(-A, A)
    denom = math.sqrt(float(head_dim * scale_factor))
    total: Optional[torch.Tensor] = None

    if "c2p" in types:
        if kr is None:
            raise RuntimeError("p2p/c2p path requires pos_key projection.")
        if variant == "einsum":
            table = torch.einsum("bhqd,hkd->bhqk", q, kr)
        else:
            qf = q.permute(1, 0, 2, 3).reshape(H, B * Lq, head_dim)
            table = torch.bmm(qf, kr.transpose(1, 2).contiguous()).reshape(H, B, Lq, 2 * A).permute(1, 0, 2, 3)
        idx = (rel + A).clamp(0, 2 * A - 1).expand(B, H, Lq, Lk)
        term = table.gather(-1, idx) / denom
        total = term if total is None else total + term

    if "p2c" in types:
        if qr is None:
            raise RuntimeError("p2p/p2c path requires pos_query projection.")
        if variant == "einsum":
            table = torch.einsum("bhkd,hqd->bhkq", k, qr)
        else:
            kf = k.permute(1, 0, 2, 3).reshape(H, B * Lk, head_dim)
            table = torch.bmm(kf, qr.transpose(1, 2).contiguous()).reshape(H, B, Lk, 2 * A).permute(1, 0, 2, 3)
        idx = (A - rel.transpose(0, 1)).clamp(0, 2 * A - 1).expand(B, H, Lk, Lq)
        term = table.gather(-1, idx).transpose(-1, -2) / denom
        total = term if total is None else total + term

    if "p2p" in types:
        if kr is None or qr is None:
            raise RuntimeError("p2p path requires both pos_key and pos_query projections.")
        pq = qr[:, A:, :]
        if pq.shape[1] == 0:
            term = torch.zeros((B, H, Lq, Lk), dtype=qr.dtype)
        else:
            tab = torch.einsum("hqd,hkd->hqk", pq, kr)
            rows = torch.arange(Lq).clamp(max=tab.shape[1] - 1)
            tab = tab.index_select(1, rows)
            idx = (rel + A).clamp(0, 2 * A - 1).expand(H, Lq, Lk)
            term = (tab.gather(-1, idx) / denom).unsqueeze(0).expand(B, H, Lq, Lk)
        total = term if total is None else total + term

    if total is None:
        total = torch.zeros((B, H, Lq, Lk), dtype=q.dtype)
    return total


# --- modeling/deberta_v2_native.py:592-652 (score / mask / softmax / PV) ------
def attend(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kr: Optional[torch.Tensor],
    qr: Optional[torch.Tensor],
    rel: Optional[torch.Tensor],
    attention_mask: Optional[torch.Tensor],
    *,
    types: list[str],
    att_span: int,
    use_relative: bool = True,
    variant: str = "einsum",
    dropout_keep: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Context ``(B, H, Lq, D)`` (in v's dtype) and probabilities.  q, k, v
    are ``(B, H, L, D)``; kr / qr ``(H, 2A, D)``; rel ``(Lq, Lk)``.
    ``dropout_keep`` (bool ``(B, H, Lq, Lk)``) with ``dropout_p``: the
    reference's attention dropout (:636) with its mask given."""
    D = q.shape[-1]
    sf = 1 + sum(t in types for t in ("c2p", "p2c", "p2p"))
    denom = math.sqrt(float(D * sf))
    # The reference scores in fp32 (query_layer.float(), :602-603); fp64
    # inputs (used only to pin this oracle) stay in fp64.
    score_dtype = torch.float64 if q.dtype == torch.float64 else torch.float32
    qf, kf = q.to(score_dtype), k.to(score_dtype)
    scores = torch.matmul(qf, kf.transpose(-1, -2)) / denom
    if use_relative and (kr is not None or qr is not None):
        kr_f = kr.to(qf.dtype) if kr is not None else None
        qr_f = qr.to(qf.dtype) if qr is not None else None
        scores = scores + relative_bias(qf, kf, kr_f, qr_f, rel, att_span, types, sf, D, variant).to(score_dtype)
    live = None
    if attention_mask is not None:
        keep = keep_mask(attention_mask)
        if keep.ndim != 4:
            raise ValueError(f"attention_mask must be rank-4 [B,1,Q,K]; got shape={tuple(keep.shape)}")
        scores = scores.masked_fill(~keep, torch.finfo(scores.dtype).min)
        if keep.shape[-2] == 1:
            live = keep.transpose(-2, -1)
        else:
            live = torch.diagonal(keep, dim1=-2, dim2=-1).unsqueeze(-1)
        scores = torch.where(live, scores, torch.zeros_like(scores))
    probs = torch.softmax(scores, dim=-1)
    if dropout_keep is not None:
        # nn.Dropout in training: kept elements scaled by 1 / (1 - p) (:636)
        probs = probs * dropout_keep.to(probs.dtype) / (1.0 - dropout_p)
    if live is not None:
        probs = probs * live.to(probs.dtype)
    probs = probs.to(v.dtype)
    return torch.matmul(probs, v), probs


# --- modeling/deberta_v2_native.py:168-296, 564-652 (the module) -------------
class EagerDisentangledSelfAttention(nn.Module):
    """Reference-shaped module: same parameter names as the reference (and as
    deberta_amd.DisentangledSelfAttention), eager forward."""

    def __init__(self, config: Any, variant: str = "einsum") -> None:
        super().__init__()
        hidden = int(config.hidden_size)
        self.num_attention_heads = int(config.num_attention_heads)
        self.attention_head_size = int(getattr(config, "attention_head_size", hidden // self.num_attention_heads))
        width = self.num_attention_heads * self.attention_head_size
        self.query_proj = nn.Linear(hidden, width)
        self.key_proj = nn.Linear(hidden, width)
        self.value_proj = nn.Linear(hidden, width)
        self.share_att_key = bool(getattr(config, "share_att_key", False))
        self.pos_att_type = pos_att_types(getattr(config, "pos_att_type", None))
        self.relative_attention = bool(getattr(config, "relative_attention", False))
        self.position_buckets = int(getattr(config, "position_buckets", -1))
        self.max_relative_positions = int(getattr(config, "max_relative_positions", -1))
        if self.max_relative_positions < 1:
            self.max_relative_positions = int(config.max_position_embeddings)
        self.pos_ebd_size = self.position_buckets if self.position_buckets > 0 else self.max_relative_positions
        self.pos_key_proj = None
        self.pos_query_proj = None
        if self.relative_attention and not self.share_att_key:
            if "c2p" in self.pos_att_type or "p2p" in self.pos_att_type:
                self.pos_key_proj = nn.Linear(hidden, width)
            if "p2c" in self.pos_att_type or "p2p" in self.pos_att_type:
                self.pos_query_proj = nn.Linear(hidden, width)
        self.variant = variant

    def heads(self, x: torch.Tensor) -> torch.Tensor:
        B, L, _ = x.shape
        return x.view(B, L, self.num_attention_heads, self.attention_head_size).permute(0, 2, 1, 3).contiguous()

    def project_rel(self, rel_embeddings: torch.Tensor, use_query: bool) -> torch.Tensor:
        A = int(self.pos_ebd_size)
        if use_query:
            layer = self.query_proj if self.share_att_key else self.pos_query_proj
        else:
            layer = self.key_proj if self.share_att_key else self.pos_key_proj
        if layer is None:
            raise RuntimeError("Requested relative projection is not configured for this attention module.")
        out = layer(rel_embeddings[: 2 * A])
        return out.view(2 * A, self.num_attention_heads, self.attention_head_size).permute(1, 0, 2).contiguous()

    def forward(
        self,
        hidden_states: torch.Tensor,
        attention_mask: Optional[torch.Tensor],
        output_attentions: bool = False,
        query_states: Optional[torch.Tensor] = None,
        relative_pos: Optional[torch.Tensor] = None,
        rel_embeddings: Optional[torch.Tensor] = None,
        dropout_keep: Optional[torch.Tensor] = None,
        dropout_p: float = 0.0,
    ) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        """The reference forward; ``dropout_keep`` / ``dropout_p``: its
        attention dropout with the mask given (``attend``)."""
        if query_states is None:
            query_states = hidden_states
        q = self.heads(self.query_proj(query_states))
        k = self.heads(self.key_proj(hidden_states))
        v = self.heads(self.value_proj(hidden_states))
        kr = qr = rel = None
        use_rel = self.relative_attention and rel_embeddings is not None
        if use_rel:
            Lq, Lk = q.shape[2], k.shape[2]
            rel = canonical_rel(relative_pos, Lq, Lk, self.position_buckets, self.max_relative_positions)
            sdt = torch.float64 if q.dtype == torch.float64 else torch.float32
            if "c2p" in self.pos_att_type or "p2p" in self.pos_att_type:
                kr = self.project_rel(rel_embeddings, use_query=False).to(sdt)
            if "p2c" in self.pos_att_type or "p2p" in self.pos_att_type:
                qr = self.project_rel(rel_embeddings, use_query=True).to(sdt)
        ctx, probs = attend(
            q, k, v, kr, qr, rel, attention_mask,
            types=self.pos_att_type, att_span=self.pos_ebd_size, use_relative=use_rel, variant=self.variant,
            dropout_keep=dropout_keep, dropout_p=dropout_p,
        )
        B, H, L, D = ctx.shape
        ctx = ctx.permute(0, 2, 1, 3).contiguous().view(B, L, H * D).to(hidden_states.dtype)
        return (ctx, probs.to(hidden_states.dtype)) if output_attentions else (ctx, None)


def make_config(**kw: Any) -> SimpleNamespace:
    """Minimal config namespace with the fields the module reads."""
    base = dict(
        hidden_size=128,
        num_attention_heads=4,
        max_position_embeddings=512,
        relative_attention=True,
        pos_att_type="c2p|p2c",
        position_buckets=256,
        max_relative_positions=512,
        share_att_key=False,
        hidden_dropout_prob=0.0,
        attention_probs_dropout_prob=0.0,
        hf_attention_kernel="dynamic",
    )
    base.update(kw)
    return SimpleNamespace(**base)
