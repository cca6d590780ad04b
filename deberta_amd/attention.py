"""Disentangled self-attention on the fused HIP kernels.

``DisentangledSelfAttention`` keeps the reference module's parameters
(``query_proj``, ``key_proj``, ``value_proj``, ``pos_key_proj``,
``pos_query_proj``), attributes and forward signature
(deberta_v2_native.py:168-222, 564-652), so a reference state dict loads
into it and an encoder calls it unchanged.  The score/softmax/PV chain and
its backward run in ``deberta_amd::dsa_fwd`` / ``dsa_bwd``.

``disentangled_attention`` is the functional form: it takes the projected
layers and relative tables directly.
"""

from __future__ import annotations

import math
from typing import Any, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.weak import WeakIdKeyDictionary

from deberta_amd import ops
from deberta_amd.config import normalize_attention_kernel, normalize_pos_att_type
from deberta_amd.masks import SegmentMask, kernel_masks, normalize_keep_mask, tensor_version
from deberta_amd.unfused import relative_terms, unfused_attention
from deberta_amd.relpos import (
    build_relative_position,
    is_monotone,
    is_toeplitz,
    normalize_relative_pos,
    relative_offset_table,
    table_from_matrix,
)

_TABLE_CACHE: dict[tuple, torch.Tensor] = {}
# relative_pos tensor -> (version, (Lq, Lk, device), verdict, offset table),
# keyed by object identity (WeakIdKeyDictionary: Tensor.__eq__ is
# elementwise and cannot decide a lookup)
_TOEPLITZ_OK: WeakIdKeyDictionary = WeakIdKeyDictionary()


def _compiling() -> bool:
    return bool(torch.compiler.is_compiling())


def canonical_table(query_len: int, key_len: int, buckets: int, max_position: int, device) -> torch.Tensor:
    """Cached int32 offset table of ``build_relative_position``."""
    if _compiling():
        return relative_offset_table(query_len, key_len, bucket_size=buckets, max_position=max_position, device=device)
    key = (int(query_len), int(key_len), int(buckets), int(max_position), str(torch.device(device)))
    t = _TABLE_CACHE.get(key)
    if t is None:
        t = relative_offset_table(query_len, key_len, bucket_size=buckets, max_position=max_position, device=device)
        _TABLE_CACHE[key] = t
    return t


def table_for(
    relative_pos: Optional[torch.Tensor],
    query_len: int,
    key_len: int,
    buckets: int,
    max_position: int,
    device,
    strict: bool = True,
) -> Optional[torch.Tensor]:
    """Offset table for the kernels from ``relative_pos`` (or the canonical
    one when it is None).  A given matrix must depend on ``i - j`` only and
    be non-decreasing in it (as every matrix build_relative_position returns);
    this is verified once per tensor object and version in eager mode (on
    every call for inference tensors, which keep no version).  A matrix that is
    not raises ``ValueError``, or returns None with ``strict=False``."""
    if relative_pos is None:
        return canonical_table(query_len, key_len, buckets, max_position, device)
    if _compiling():
        return table_from_matrix(normalize_relative_pos(relative_pos.to(device), query_len, key_len))
    # The verdict (and the table) is kept per caller tensor object and
    # version: a temporary made from it (a cast, a copy to the device) may
    # reuse a freed block of another matrix, so no address can key it.
    version = tensor_version(relative_pos)
    where = (int(query_len), int(key_len), str(torch.device(device)))
    hit = _TOEPLITZ_OK.get(relative_pos) if version is not None else None
    if hit is not None and hit[0] == version and hit[1] == where:
        ok, table = hit[2], hit[3]
    else:
        rp = normalize_relative_pos(relative_pos.to(device), query_len, key_len)
        table = table_from_matrix(rp)
        ok = is_toeplitz(rp, table) and is_monotone(table)
        if version is not None:
            _TOEPLITZ_OK[relative_pos] = (version, where, ok, table)
    if not ok:
        if not strict:
            return None
        raise ValueError(
            "relative_pos must depend on i - j only and be non-decreasing in it "
            "(as build_relative_position produces) for the fused disentangled-attention kernels"
        )
    return table


# The kernels' forms: element types and head dims (anything else runs the
# torch path, as the reference runs every dtype and head dim)
_KERNEL_DTYPES = (torch.float32, torch.bfloat16)
_KERNEL_HEAD_DIMS = (32, 64)


def _kernel_form(t: torch.Tensor, head_dim: int) -> bool:
    return t.device.type == "cuda" and t.dtype in _KERNEL_DTYPES and int(head_dim) in _KERNEL_HEAD_DIMS


def _require_gpu(t: torch.Tensor) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"fused disentangled attention runs on the GPU (HIP) only; got a tensor on {t.device}"
        )


def _relative_matrix(
    relative_pos: Optional[torch.Tensor], query_len: int, key_len: int, buckets: int, max_position: int, device
) -> torch.Tensor:
    """The ``(Lq, Lk)`` relative positions the reference's score terms use:
    ``build_relative_position`` when None, else the given matrix with the
    reference's rank handling (deberta_v2_native.py:235-271), as given."""
    if relative_pos is None:
        return build_relative_position(query_len, key_len, bucket_size=buckets, max_position=max_position, device=device)
    return normalize_relative_pos(relative_pos.to(device), query_len, key_len)


def _dense_keep(attention_mask, device) -> Optional[torch.Tensor]:
    """The rank-4 boolean keep mask of ``attention_mask`` (None, a keep mask
    or a ``SegmentMask``) for the torch-operation path."""
    if attention_mask is None:
        return None
    if isinstance(attention_mask, SegmentMask):
        return attention_mask.dense().to(device)
    keep = normalize_keep_mask(attention_mask)
    if keep.ndim != 4:
        raise ValueError(f"attention_mask must be rank-4 [B,1,Q,K]; got shape={tuple(keep.shape)}")
    return keep


def _check_mask_rank(attention_mask) -> None:
    """The reference's mask contract (mask_utils.py:8-32 and the rank check
    of deberta_v2_native.py:619-623), checked without replacing the caller's
    tensor: per-mask checks are cached on the caller's object."""
    if attention_mask is None or isinstance(attention_mask, SegmentMask):
        return
    if not isinstance(attention_mask, torch.Tensor) or torch.is_floating_point(attention_mask):
        normalize_keep_mask(attention_mask)  # raises the reference's TypeError / ValueError
    if attention_mask.ndim != 4:
        raise ValueError(f"attention_mask must be rank-4 [B,1,Q,K]; got shape={tuple(attention_mask.shape)}")


def position_query_rows(qr: torch.Tensor, query_len: int, att_span: int) -> torch.Tensor:
    """The p2p term's query rows ``Qr[:, A + min(i, A - 1)]`` for i <
    query_len, as ``[1, Lq, H, D]`` (deberta_v2_native.py:330-342:
    the positive half of the pos-query table, indexed by the clamped query
    position).  The gather runs in fp32, so that its backward sums the
    gradients of the rows that share a table row (every query past A - 1
    reads row 2A - 1) in fp32 and rounds once, where a bf16 scatter-add
    rounded after every addition."""
    A = int(att_span)
    rows = torch.arange(query_len, device=qr.device).clamp(max=A - 1) + A
    return qr.float().index_select(1, rows).permute(1, 0, 2).unsqueeze(0).to(qr.dtype)


def relative_operands(
    types: list[str],
    q: torch.Tensor,
    kr: Optional[torch.Tensor],
    qr: Optional[torch.Tensor],
    att_span: int,
) -> tuple[Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor]]:
    """The kernels' relative operands ``(kr, qr, qc)`` for the score terms in
    ``types`` (q ``[B, L, H, D]``; kr / qr the projected ``(H, 2A, D)``
    tables in q's dtype).

    The p2p term, ``Qr[A + min(i, A - 1)] . Kr[c(i - j)]``, reads the same
    Kr rows as c2p, so it is carried by the c2p term's query rows:
    ``qc = q + Qr[A + min(i, A - 1)]`` with c2p, ``qc = Qr[A + min(i, A - 1)]``
    alone without it (the kernels then run their c2p term on qc).  Autograd
    returns qc's gradient to q and to Qr."""
    c2p, p2c, p2p = ("c2p" in types), ("p2c" in types), ("p2p" in types)
    if (c2p or p2p) and kr is None:
        raise RuntimeError("p2p/c2p path requires pos_key projection.")
    if (p2c or p2p) and qr is None:
        raise RuntimeError("p2p/p2c path requires pos_query projection.")
    if p2p and (kr is None or qr is None):
        raise RuntimeError("p2p path requires both pos_key and pos_query projections.")
    qc = None
    if p2p:
        pq = position_query_rows(qr, q.shape[1], att_span)
        qc = q + pq if c2p else pq.expand(q.shape[0], -1, -1, -1)
    return (kr if (c2p or p2p) else None), (qr if p2c else None), qc


def fused_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    kr: Optional[torch.Tensor],
    qr: Optional[torch.Tensor],
    table: Optional[torch.Tensor],
    attention_mask: Optional[torch.Tensor],
    att_span: int,
    scale: float,
    qc: Optional[torch.Tensor] = None,
    qkv: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
) -> torch.Tensor:
    """Core call on ``[B, L, H, D]`` layers; returns ``[B, Lq, H, D]``.
    ``kr`` / ``qr`` are the c2p / p2c tables (None: term off); ``qc`` the
    c2p term's query rows (None: q).  ``qkv``: q, k and v packed as one
    ``[B, L, 3, H, D]`` tensor (q, k, v are then None); the op takes it
    whole and its gradient comes back as one tensor.  ``dropout_p``:
    attention dropout in the kernels, with a fresh seed from torch's CPU
    generator (``ops.dropout_threshold(dropout_p)`` must lie in [1, 65535])."""
    ref = qkv if qkv is not None else q  # shapes, dtype and device
    _require_gpu(ref)
    B, Lq, H = ref.shape[0], ref.shape[1], ref.shape[-2]
    Lk = Lq if qkv is not None else k.shape[1]
    key_keep, pair_keep = kernel_masks(attention_mask, B, Lq, Lk, ref.device, heads=H)
    if kr is not None:
        kr = kr.to(ref.dtype)
    if qr is not None:
        qr = qr.to(ref.dtype)
    if qc is not None:
        qc = qc.to(ref.dtype)
    if kr is None and qr is None:
        table = None
    # The relative term is saved only when a backward can follow.
    save_bias = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v, qkv, kr, qr, qc)
    )
    drop_t, seed = 0, None
    if dropout_p > 0.0:
        drop_t = ops.dropout_threshold(dropout_p)
        if not 0 < drop_t < 65536:
            raise ValueError(f"dropout_p={dropout_p} has no kernel form (threshold {drop_t} outside [1, 65535])")
        seed = ops.draw_dropout_seed()
    if qkv is not None:
        out, _, _, _ = ops.attention_packed(
            qkv, kr, qr, table, key_keep, pair_keep, int(att_span), float(scale), save_bias, qc, drop_t, seed
        )
    else:
        out, _, _, _ = ops.attention(
            q, k, v, kr, qr, table, key_keep, pair_keep, int(att_span), float(scale), save_bias, qc, drop_t, seed
        )
    return out


def disentangled_attention(
    query_layer: torch.Tensor,
    key_layer: torch.Tensor,
    value_layer: torch.Tensor,
    pos_key_layer: Optional[torch.Tensor],
    pos_query_layer: Optional[torch.Tensor],
    relative_pos: Optional[torch.Tensor],
    attention_mask: Optional[torch.Tensor],
    *,
    position_buckets: int,
    max_relative_positions: int,
    att_type: Any = "c2p|p2c",
    scale_factor: Optional[int] = None,
    layout: str = "bhld",
    dropout_p: float = 0.0,
) -> torch.Tensor:
    """Fused disentangled attention on already-projected layers.

    ``query/key/value_layer`` are ``(B, H, L, D)`` (``layout="bhld"``, the
    reference's ``_shape`` output) or ``(B, L, H, D)`` (``layout="blhd"``, the
    Linear output viewed per head, read in place).  ``pos_key_layer`` /
    ``pos_query_layer`` are the projected relative tables ``(H, 2A, D)``
    (``_project_rel``); the c2p / p2c / p2p terms are used when ``att_type``
    names them.  ``relative_pos`` and ``attention_mask`` follow the module's
    contract.  ``scale_factor`` defaults to ``1 + #att_type terms``.
    ``dropout_p``: attention dropout on the probabilities (applied as
    given: the caller decides whether it is training), in the kernels when
    its threshold (``ops.dropout_threshold``) is in [1, 65535], else with
    torch's dropout on the torch path.  The result has the layout of
    ``query_layer``.
    """
    types = normalize_pos_att_type(att_type)
    if layout not in ("bhld", "blhd"):
        raise ValueError(f"layout must be 'bhld' or 'blhd', got {layout!r}")
    if layout == "bhld":
        q, k, v = (t.transpose(1, 2) for t in (query_layer, key_layer, value_layer))
    else:
        q, k, v = query_layer, key_layer, value_layer
    if scale_factor is None:
        scale_factor = 1 + sum(t in types for t in ("c2p", "p2c", "p2p"))
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(float(D * scale_factor))
    tables = [t for t in (pos_key_layer, pos_query_layer) if t is not None]
    att_span = tables[0].shape[1] // 2 if tables else 1
    in_kernels = (dropout_p <= 0.0 or 0 < ops.dropout_threshold(dropout_p) < 65536) and _kernel_form(q, D)
    if not in_kernels:
        # CPU tensors, dtypes and head dims the kernels do not take, and a
        # dropout probability they cannot draw: the same chain in torch
        # operations (deberta_amd.unfused)
        rel_pos = None
        if any(t in types for t in ("c2p", "p2c", "p2p")):
            rel_pos = _relative_matrix(
                relative_pos, q.shape[1], k.shape[1], position_buckets, max_relative_positions, q.device
            )
        out, _ = unfused_attention(
            q, k, v, pos_key_layer, pos_query_layer, rel_pos, _dense_keep(attention_mask, q.device),
            att_span, scale, types, nn.Dropout(dropout_p) if dropout_p > 0.0 else None,
        )
        return out.transpose(1, 2) if layout == "bhld" else out
    kr, qr, qc = relative_operands(
        types, q,
        None if pos_key_layer is None else pos_key_layer.to(q.dtype),
        None if pos_query_layer is None else pos_query_layer.to(q.dtype),
        att_span,
    )
    table = None
    if kr is not None or qr is not None:
        table = table_for(relative_pos, q.shape[1], k.shape[1], position_buckets, max_relative_positions, q.device)
    _check_mask_rank(attention_mask)
    out = fused_attention(q, k, v, kr, qr, table, attention_mask, att_span, scale, qc, dropout_p=dropout_p)
    return out.transpose(1, 2) if layout == "bhld" else out


class DisentangledSelfAttention(nn.Module):
    """DeBERTa-v2 disentangled self-attention on the fused HIP kernels.

    Construction mirrors deberta_v2_native.py:171-222 (same parameter names
    and shapes, same config attributes read with the same defaults).
    """

    def __init__(self, config: Any) -> None:
        super().__init__()
        hidden_size = int(config.hidden_size)
        num_heads = int(config.num_attention_heads)
        if hidden_size % num_heads != 0:
            raise ValueError(
                f"hidden_size ({hidden_size}) must be divisible by num_attention_heads ({num_heads})."
            )
        self.num_attention_heads = num_heads
        self.attention_head_size = int(getattr(config, "attention_head_size", hidden_size // num_heads))
        self.all_head_size = self.num_attention_heads * self.attention_head_size

        self.query_proj = nn.Linear(hidden_size, self.all_head_size, bias=True)
        self.key_proj = nn.Linear(hidden_size, self.all_head_size, bias=True)
        self.value_proj = nn.Linear(hidden_size, self.all_head_size, bias=True)

        self.share_att_key = bool(getattr(config, "share_att_key", False))
        self.pos_att_type = normalize_pos_att_type(getattr(config, "pos_att_type", None))
        self.relative_attention = bool(getattr(config, "relative_attention", False))

        self.position_buckets = int(getattr(config, "position_buckets", -1))
        self.max_relative_positions = int(getattr(config, "max_relative_positions", -1))
        if self.max_relative_positions < 1:
            self.max_relative_positions = int(config.max_position_embeddings)

        self.pos_ebd_size = self.max_relative_positions
        if self.position_buckets > 0:
            self.pos_ebd_size = self.position_buckets

        self.pos_dropout = nn.Dropout(float(getattr(config, "hidden_dropout_prob", 0.0)))
        self.attn_kernel = normalize_attention_kernel(getattr(config, "hf_attention_kernel", "dynamic"))

        if self.relative_attention and (not self.share_att_key):
            if ("c2p" in self.pos_att_type) or ("p2p" in self.pos_att_type):
                self.pos_key_proj = nn.Linear(hidden_size, self.all_head_size, bias=True)
            else:
                self.pos_key_proj = None
            if ("p2c" in self.pos_att_type) or ("p2p" in self.pos_att_type):
                self.pos_query_proj = nn.Linear(hidden_size, self.all_head_size, bias=True)
            else:
                self.pos_query_proj = None
        else:
            self.pos_key_proj = None
            self.pos_query_proj = None

        self.dropout = nn.Dropout(float(getattr(config, "attention_probs_dropout_prob", 0.0)))

    def _heads(self, x: torch.Tensor) -> torch.Tensor:
        """``(B, L, H*D)`` Linear output -> ``(B, L, H, D)`` view (no copy)."""
        bsz, seq_len, _ = x.shape
        return x.view(bsz, seq_len, self.num_attention_heads, self.attention_head_size)

    def _project_qkv(
        self, hidden_states: torch.Tensor, query_states: Optional[torch.Tensor]
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
        """(q, k, v, qkv): one fused projection (deberta_v2_native.py:587-589
        as a single GEMM) as ``qkv`` ``(B, L, 3, H, D)``, with q, k, v None
        (callers that need them take ``qkv.unbind(2)``: where they reach
        autograd separately their gradient is one stack, where three
        ``select``s zero-filled and copied three ``(B, L, 3 H D)`` tensors and
        added them).  The three weights are concatenated at call time, so
        the parameters (and the state-dict keys query_proj / key_proj /
        value_proj) stay the reference's.  With separate ``query_states``
        only the key and value projections are fused, and q, k, v are
        ``(B, L, H, D)`` views (qkv None)."""
        H, D = self.num_attention_heads, self.attention_head_size
        bsz, seq_len, _ = hidden_states.shape
        if query_states is None:
            w = torch.cat([self.query_proj.weight, self.key_proj.weight, self.value_proj.weight])
            bias = torch.cat([self.query_proj.bias, self.key_proj.bias, self.value_proj.bias])
            return None, None, None, F.linear(hidden_states, w, bias).view(bsz, seq_len, 3, H, D)
        q = self._heads(self.query_proj(query_states))
        w = torch.cat([self.key_proj.weight, self.value_proj.weight])
        bias = torch.cat([self.key_proj.bias, self.value_proj.bias])
        k, v = F.linear(hidden_states, w, bias).view(bsz, seq_len, 2, H, D).unbind(2)
        return q, k, v, None

    def _project_rel(self, rel_embeddings: torch.Tensor, *, use_query: bool) -> torch.Tensor:
        """Projected relative table ``(H, 2A, D)`` as a view of the Linear
        output (deberta_v2_native.py:273-296 without the permute copy)."""
        att_span = int(self.pos_ebd_size)
        rel = rel_embeddings[: 2 * att_span, :]
        if use_query:
            proj_layer = self.query_proj if self.share_att_key else self.pos_query_proj
        else:
            proj_layer = self.key_proj if self.share_att_key else self.pos_key_proj
        if proj_layer is None:
            raise RuntimeError("Requested relative projection is not configured for this attention module.")
        projected = proj_layer(rel)
        projected = projected.view(2 * att_span, self.num_attention_heads, self.attention_head_size)
        return projected.permute(1, 0, 2)

    def _relative_tables(
        self, rel_embeddings: torch.Tensor, dtype: torch.dtype
    ) -> tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """(Kr, Qr) projected for the configured terms (None where unused),
        in ``dtype`` (deberta_v2_native.py:372-375).  When both are needed
        they come from one GEMM through the two weight matrices
        concatenated at call time (the parameters stay the reference's), as
        ``(H, 2A, D)`` views of its output."""
        types = self.pos_att_type
        need_k = ("c2p" in types) or ("p2p" in types)
        need_q = ("p2c" in types) or ("p2p" in types)
        if need_k and need_q:
            kl = self.key_proj if self.share_att_key else self.pos_key_proj
            ql = self.query_proj if self.share_att_key else self.pos_query_proj
            if kl is None or ql is None:
                raise RuntimeError("Requested relative projection is not configured for this attention module.")
            A, H, D = int(self.pos_ebd_size), self.num_attention_heads, self.attention_head_size
            w = torch.cat([kl.weight, ql.weight])
            b = torch.cat([kl.bias, ql.bias])
            kr, qr = F.linear(rel_embeddings[: 2 * A, :], w, b).to(dtype).view(2 * A, 2, H, D).unbind(1)
            return kr.permute(1, 0, 2), qr.permute(1, 0, 2)
        kr = self._project_rel(rel_embeddings, use_query=False).to(dtype) if need_k else None
        qr = self._project_rel(rel_embeddings, use_query=True).to(dtype) if need_q else None
        return kr, qr

    def disentangled_attention_bias(
        self,
        query_layer: torch.Tensor,
        key_layer: torch.Tensor,
        relative_pos: Optional[torch.Tensor],
        rel_embeddings: torch.Tensor,
        scale_factor: int,
    ) -> torch.Tensor:
        """The relative score term ``(c2p + p2c + p2p) / sqrt(D * scale_factor)``
        of ``(B, H, Q, D)`` query and key layers, as ``(B, H, Q, K)`` in the
        query's dtype (deberta_v2_native.py:530-562; every kernel choice
        computes the same function).  Computed by the fused kernels' band
        code (``deberta_amd::dsa_bias``), unmasked; forward only (training
        differentiates through ``forward``).  CPU tensors take the same
        terms in torch operations (``deberta_amd.unfused.relative_terms``)."""
        if not _kernel_form(query_layer, query_layer.shape[-1]):
            return self._bias_unfused(query_layer, key_layer, relative_pos, rel_embeddings, scale_factor)
        q = query_layer.transpose(1, 2)
        k = key_layer.to(q.dtype).transpose(1, 2)
        Lq, Lk = q.shape[1], k.shape[1]
        att_span = int(self.pos_ebd_size)
        kr_full, qr_full = self._relative_tables(rel_embeddings, q.dtype)
        kr, qr, qc = relative_operands(self.pos_att_type, q, kr_full, qr_full, att_span)
        table = None
        if kr is not None or qr is not None:
            table = table_for(
                relative_pos, Lq, Lk, self.position_buckets, self.max_relative_positions, q.device, strict=False
            )
            if table is None:  # not a function of i - j: used as given
                return self._bias_unfused(query_layer, key_layer, relative_pos, rel_embeddings, scale_factor)
        scale = 1.0 / math.sqrt(float(self.attention_head_size * int(scale_factor)))
        return torch.ops.deberta_amd.dsa_bias(q, k, kr, qr, table, att_span, scale, qc)

    def _bias_unfused(
        self,
        query_layer: torch.Tensor,
        key_layer: torch.Tensor,
        relative_pos: Optional[torch.Tensor],
        rel_embeddings: torch.Tensor,
        scale_factor: int,
    ) -> torch.Tensor:
        """``disentangled_attention_bias`` in torch operations (CPU tensors,
        other dtypes and head dims, a ``relative_pos`` used as given)."""
        Lq, Lk = query_layer.shape[2], key_layer.shape[2]
        kr, qr = self._relative_tables(rel_embeddings, query_layer.dtype)
        rel_pos = None
        if any(t in self.pos_att_type for t in ("c2p", "p2c", "p2p")):
            rel_pos = _relative_matrix(
                relative_pos, Lq, Lk, self.position_buckets, self.max_relative_positions, query_layer.device
            )
        scale = 1.0 / math.sqrt(float(self.attention_head_size * int(scale_factor)))
        qh, kh = query_layer.float(), key_layer.float()
        rel = relative_terms(qh, kh, kr, qr, rel_pos, int(self.pos_ebd_size), scale, self.pos_att_type)
        if rel is None:
            return torch.zeros(
                (qh.shape[0], qh.shape[1], Lq, Lk), device=query_layer.device, dtype=query_layer.dtype
            )
        return rel.to(query_layer.dtype)

    def forward(
        self,
        hidden_states: torch.Tensor,
        attention_mask: Optional[torch.Tensor],
        output_attentions: bool = False,
        query_states: Optional[torch.Tensor] = None,
        relative_pos: Optional[torch.Tensor] = None,
        rel_embeddings: Optional[torch.Tensor] = None,
    ) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Same contract as the reference forward (deberta_v2_native.py:564-652).

        The fused kernels run the call, attention dropout in training
        included (the kernels draw the keep bits, ``deberta_amd.ops``),
        unless it is on CPU tensors, in a dtype other than float32 /
        bfloat16 or with a head dim other than 32 / 64, needs the
        probabilities themselves (``output_attentions=True``), its
        ``relative_pos`` does not depend on ``i - j`` alone, or its dropout
        probability has no kernel form (below 2^-17 or above 1 - 2^-17);
        those run the same chain in torch
        operations on the tensors' device (``deberta_amd.unfused``, with
        torch's dropout) and return the probabilities when asked.
        """
        drop_p = float(self.dropout.p) if self.training else 0.0
        drop_in_kernels = drop_p <= 0.0 or 0 < ops.dropout_threshold(drop_p) < 65536

        q, k, v, qkv = self._project_qkv(hidden_states, query_states)
        model_dtype = hidden_states.dtype
        ref = qkv if qkv is not None else q  # dtype and device of the layers
        unfused = (not _kernel_form(ref, self.attention_head_size)) or output_attentions or not drop_in_kernels
        Lq = ref.shape[1]
        Lk = Lq if qkv is not None else k.shape[1]

        scale_factor = 1 + sum(t in self.pos_att_type for t in ("c2p", "p2c", "p2p"))
        scale = 1.0 / math.sqrt(float(self.attention_head_size * scale_factor))

        kr = qr = qc = table = kr_full = qr_full = None
        att_span = 1
        relative = self.relative_attention and rel_embeddings is not None
        if relative:
            rel_embeddings = self.pos_dropout(rel_embeddings)
            att_span = int(self.pos_ebd_size)
            kr_full, qr_full = self._relative_tables(rel_embeddings, ref.dtype)
            if not unfused:
                # p2p's query rows add to q: only then is q needed on its own
                qp = q if q is not None or "p2p" not in self.pos_att_type else qkv.unbind(2)[0]
                kr, qr, qc = relative_operands(self.pos_att_type, qp, kr_full, qr_full, att_span)
                if kr is not None or qr is not None:
                    table = table_for(
                        relative_pos,
                        Lq,
                        Lk,
                        self.position_buckets,
                        self.max_relative_positions,
                        ref.device,
                        strict=False,
                    )
                    unfused = table is None  # not a function of i - j: used as given
        if unfused:
            if qkv is not None:
                q, k, v = qkv.unbind(2)
            return self._forward_unfused(
                q, k, v, kr_full, qr_full, relative_pos if relative else None, relative, attention_mask,
                att_span, scale, model_dtype, output_attentions,
            )

        _check_mask_rank(attention_mask)

        # the op takes the packed projection whole (its gradient comes back
        # as one tensor)
        ctx = fused_attention(q, k, v, kr, qr, table, attention_mask, att_span, scale, qc, qkv=qkv, dropout_p=drop_p)
        bsz, seq_len = ctx.shape[0], ctx.shape[1]
        context_layer = ctx.reshape(bsz, seq_len, self.all_head_size).to(dtype=model_dtype)
        return context_layer, None

    def _forward_unfused(
        self, q, k, v, kr, qr, relative_pos, relative, attention_mask, att_span, scale, model_dtype, output_attentions
    ) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
        """The torch-operation path (``deberta_amd.unfused``) with the
        module's relative positions, mask and dropout."""
        Lq, Lk = q.shape[1], k.shape[1]
        rel_pos = None
        types = self.pos_att_type if relative else []
        if relative and any(t in types for t in ("c2p", "p2c", "p2p")):
            rel_pos = _relative_matrix(
                relative_pos, Lq, Lk, self.position_buckets, self.max_relative_positions, q.device
            )
        keep = _dense_keep(attention_mask, q.device)
        ctx, probs = unfused_attention(
            q, k, v, kr, qr, rel_pos, keep, att_span, scale, types, self.dropout if self.training else None
        )
        context_layer = ctx.reshape(ctx.shape[0], Lq, self.all_head_size).to(dtype=model_dtype)
        if not output_attentions:
            return context_layer, None
        return context_layer, probs.to(v.dtype).to(model_dtype)
