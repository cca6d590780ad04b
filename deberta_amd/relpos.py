"""Relative-position ids for disentangled attention, and their 1-D table form.

The reference builds a full ``(Lq, Lk)`` matrix of bucketed ``i - j``
(deberta_v2_native.py:51-112).  Every entry depends on ``i - j`` only, so the
kernels take the ``Lq + Lk - 1`` distinct values as a 1-D int32 table:
``table[(i - j) + (Lk - 1)]``.  The table is computed with the same torch
operations as the matrix, on the device the attention runs on, so the
bucket values (including the fp32 ``log``/``ceil`` at the saturation edge)
are the ones the reference would produce there.
"""

from __future__ import annotations

import math
from typing import Optional

import torch


def make_log_bucket_position(relative_pos: torch.Tensor, bucket_size: int, max_position: int) -> torch.Tensor:
    """Log-bucket compression of relative offsets.

    Same contract as the reference's ``_make_log_bucket_position``
    (deberta_v2_native.py:51-84): clamp to ``±(max_position - 1)``, keep
    ``|d| < bucket_size // 2`` as is, compress the rest logarithmically in
    fp32, identity when ``bucket_size // 2 <= 1`` or the log base is not
    positive.
    """
    rel = relative_pos
    if int(max_position) > 0:
        rel = rel.clamp(min=-int(max_position) + 1, max=int(max_position) - 1)
    sign = torch.sign(rel)
    mid = int(bucket_size // 2)
    if mid <= 1:
        return rel
    abs_pos = rel.abs().clamp_min(1)
    near = abs_pos < mid
    log_base = math.log(max(float(max_position - 1), float(mid + 1)) / float(mid))
    if log_base <= 0.0:
        return rel
    log_pos = torch.ceil(torch.log(abs_pos.float() / float(mid)) / log_base * float(mid - 1)) + float(mid)
    bucket = torch.where(near, abs_pos.to(log_pos.dtype), log_pos)
    bucket = bucket * sign.to(bucket.dtype)
    return bucket.to(torch.long)


def build_relative_position(
    query_len: int,
    key_len: int,
    *,
    bucket_size: int,
    max_position: int,
    device: torch.device | str | None = None,
) -> torch.Tensor:
    """``(query_len, key_len)`` matrix of (bucketed) ``i - j``, as the
    reference's ``build_relative_position`` (deberta_v2_native.py:87-112)."""
    q_ids = torch.arange(int(query_len), dtype=torch.long, device=device)
    k_ids = torch.arange(int(key_len), dtype=torch.long, device=device)
    rel = q_ids[:, None] - k_ids[None, :]
    if int(bucket_size) > 0 and int(max_position) > 0:
        rel = make_log_bucket_position(rel, int(bucket_size), int(max_position))
    return rel.to(torch.long)


def relative_offset_table(
    query_len: int,
    key_len: int,
    *,
    bucket_size: int,
    max_position: int,
    device: torch.device | str | None = None,
) -> torch.Tensor:
    """int32 table ``t[(i - j) + (key_len - 1)]`` of the matrix
    ``build_relative_position`` returns, without materialising it."""
    d = torch.arange(-(int(key_len) - 1), int(query_len), dtype=torch.long, device=device)
    if int(bucket_size) > 0 and int(max_position) > 0:
        d = make_log_bucket_position(d, int(bucket_size), int(max_position))
    return d.to(torch.int32).contiguous()


def normalize_relative_pos(relative_pos: torch.Tensor, query_len: int, key_len: int) -> torch.Tensor:
    """Canonical ``(query_len, key_len)`` long matrix from a user-given
    ``relative_pos``, with the reference's rank handling
    (deberta_v2_native.py:257-271): rank 4 uses ``[0, 0]``, rank 3 uses
    ``[0]``, other ranks but 2 raise."""
    rp = relative_pos.to(dtype=torch.long)
    if rp.ndim == 4:
        rp = rp[0, 0]
    elif rp.ndim == 3:
        rp = rp[0]
    elif rp.ndim != 2:
        raise ValueError(f"relative_pos must be rank-2/3/4, got rank={rp.ndim}")
    if rp.shape[0] != query_len or rp.shape[1] != key_len:
        rp = rp[:query_len, :key_len]
    return rp


def table_from_matrix(rp: torch.Tensor) -> torch.Tensor:
    """1-D table of a ``(Lq, Lk)`` relative-position matrix: its first row
    (offsets ``-(Lk-1)..0``, reversed) followed by the rest of its first
    column (offsets ``1..Lq-1``).  Exact when the matrix is Toeplitz."""
    first_row = rp[0, :].flip(0)
    first_col = rp[1:, 0]
    return torch.cat([first_row, first_col]).to(torch.int32).contiguous()


def is_toeplitz(rp: torch.Tensor, table: Optional[torch.Tensor] = None) -> bool:
    """True if ``rp[i, j]`` depends on ``i - j`` only.  Synchronises with the
    device (one reduction)."""
    Lq, Lk = rp.shape
    if table is None:
        table = table_from_matrix(rp)
    idx = (
        torch.arange(Lq, device=rp.device)[:, None] - torch.arange(Lk, device=rp.device)[None, :] + (Lk - 1)
    )
    return bool(torch.equal(table.to(torch.long)[idx], rp.to(torch.long)))


def is_monotone(table: torch.Tensor) -> bool:
    """True if the offset table is non-decreasing in i - j (every bucketed or
    plain relative-position table is).  Synchronises with the device."""
    t = table.to(torch.long)
    return bool((t[1:] >= t[:-1]).all()) if t.numel() > 1 else True
