"""Keep-mask contract of the attention (bool/int keep masks, float rejected),
and its translation into the byte masks the kernels read.

Mirrors ``normalize_keep_mask`` (mask_utils.py:8-32), the encoder's
``get_attention_mask`` (deberta_v2_native.py:1049-1068) and the packed
document mask ``_build_doc_block_mask`` (training/compile.py:310-349).
"""

from __future__ import annotations

from typing import Optional

import torch
from torch.utils.weak import WeakIdKeyDictionary


def tensor_version(t: torch.Tensor) -> Optional[int]:
    """``t``'s version counter (bumped by every in-place write), or None for
    an inference tensor, which keeps none: results cached per tensor object
    are then recomputed on every call."""
    return None if t.is_inference() else t._version


def normalize_keep_mask(mask: torch.Tensor, *, name: str = "attention_mask") -> torch.Tensor:
    """Bool keep mask: bool passes through, integers become ``!= 0``, floating
    masks raise ``ValueError`` and non-tensors ``TypeError`` (same messages as
    the reference)."""
    if not isinstance(mask, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(mask)!r}.")
    if mask.dtype == torch.bool:
        return mask
    if torch.is_floating_point(mask):
        raise ValueError(
            f"{name} must be a bool/integer keep-mask tensor. "
            "Floating-point masks are ambiguous (0/1 keep vs 0/-inf additive)."
        )
    return mask.ne(0)


def get_attention_mask(attention_mask: torch.Tensor) -> torch.Tensor:
    """Encoder-side canonical 4-D keep mask: ``(B,S) -> (B,1,1,S)``,
    ``(B,S,S) -> (B,1,S,S)``, ``(B,H,..) -> any over heads``."""
    mask = normalize_keep_mask(attention_mask)
    if mask.ndim <= 2:
        return mask[:, None, None, :]
    if mask.ndim == 3:
        return mask.unsqueeze(1)
    if mask.ndim == 4:
        if mask.shape[1] == 1:
            return mask
        return mask.any(dim=1, keepdim=True)
    raise ValueError(f"attention_mask must be rank-2/3/4; got rank={mask.ndim}")


def build_doc_block_mask(doc_ids: torch.Tensor) -> torch.Tensor:
    """Pairwise ``(B, S, S)`` keep mask for packed documents: active tokens
    (``doc_id != 0``) attend within their document, the diagonal marks query
    activity, and pad queries keep one edge to key 0 (CLS)."""
    if doc_ids.ndim != 2:
        raise ValueError(f"doc_ids must be rank-2 (B,S); got shape={tuple(doc_ids.shape)}")
    seq_len = int(doc_ids.shape[1])
    device = doc_ids.device
    eye = torch.eye(seq_len, dtype=torch.bool, device=device)
    cls_key = torch.zeros(seq_len, dtype=torch.bool, device=device)
    cls_key[0] = True
    active = doc_ids.ne(0)
    same_doc = doc_ids[:, :, None].eq(doc_ids[:, None, :])
    keep = same_doc & active[:, :, None] & active[:, None, :]
    keep = keep | ((~active)[:, :, None] & cls_key[None, None, :])
    keep = (keep & ~eye[None, :, :]) | (eye[None, :, :] & active[:, :, None])
    return keep


class SegmentMask:
    """Compact form of the packed-document keep mask: the ``(B, S)`` document
    id of every token (0 for padding) in place of the ``(B, 1, S, S)``
    boolean tensor ``_build_doc_block_mask`` builds (training/compile.py:
    310-349; ``build_doc_block_mask`` here).

    Accepted as ``attention_mask`` by ``DisentangledSelfAttention`` and
    ``disentangled_attention``: the kernels read the ids (4 bytes a token
    instead of S bytes) and skip the key tiles of other documents.  The
    results are those of ``dense()``, the reference's boolean mask: its pad
    queries are dead rows (their one kept key, the CLS edge, never reaches
    an output), so a pair is kept iff both tokens carry the same nonzero id.
    """

    def __init__(self, doc_ids: torch.Tensor):
        if not isinstance(doc_ids, torch.Tensor):
            raise TypeError(f"doc_ids must be a torch.Tensor, got {type(doc_ids)!r}.")
        if doc_ids.ndim != 2:
            raise ValueError(f"doc_ids must be rank-2 (B,S); got shape={tuple(doc_ids.shape)}")
        if doc_ids.dtype == torch.bool or torch.is_floating_point(doc_ids):
            raise ValueError(f"doc_ids must be an integer tensor; got {doc_ids.dtype}")
        self.doc_ids = doc_ids

    @property
    def shape(self) -> tuple[int, int, int, int]:
        b, s = self.doc_ids.shape
        return (b, 1, s, s)

    def dense(self) -> torch.Tensor:
        """The reference's ``(B, 1, S, S)`` boolean keep mask."""
        return build_doc_block_mask(self.doc_ids)[:, None]

    def segment_ids(self, device: torch.device) -> torch.Tensor:
        """``int32 [B, S]`` ids on ``device`` (the kernels' ``seg``)."""
        ids = self.doc_ids
        if ids.dtype != torch.int32:
            if ids.numel() and (int(ids.max()) > 2**31 - 1 or int(ids.min()) < -(2**31)):
                raise ValueError("doc_ids must fit in int32")
            ids = ids.to(torch.int32)
        return ids.to(device).contiguous()


def dense_as_segments(pair_keep: torch.Tensor) -> Optional[torch.Tensor]:
    """Segment ids with the same meaning as a dense ``[B, L, L]`` keep mask,
    or None if there are none.

    The kernels' segment rule keeps (i, j) iff seg_i != 0 and seg_i ==
    seg_j, and a query with seg 0 is a dead row; the dense rule keeps (i, j)
    per element, a query whose diagonal is unset being a dead row.  Take
    seg_i = 1 + (the first key row i keeps) for live rows, 0 for dead ones:
    the two rules agree iff every live row keeps exactly the keys with its
    own id (dead rows' contents never reach an output).  The packed-document
    masks of the reference (``_build_doc_block_mask``, training/compile.py:
    310-349) have this form.  One pass over the mask on its device, and one
    host synchronisation for the answer."""
    keep = pair_keep.bool()
    b, lq, lk = keep.shape
    if lq != lk or lk > 32768:
        return None
    live = keep.diagonal(dim1=1, dim2=2)
    first = keep.to(torch.uint8).argmax(dim=-1)  # first kept key (argmax: first of the maxima)
    ids = torch.where(live, first + 1, torch.zeros_like(first)).to(torch.int32)
    expect = ids[:, :, None] == ids[:, None, :]
    agree = (keep == expect) | ~live[:, :, None]
    if not bool(agree.all()):
        return None
    return ids.contiguous()


# dense mask -> (its version, segment ids or None), per mask tensor object.
# Keyed by object identity: a plain WeakKeyDictionary compares tensor keys
# with Tensor.__eq__ (elementwise), which cannot decide a lookup.
_SEGMENTS_OF: WeakIdKeyDictionary = WeakIdKeyDictionary()


def _segments_cached(mask: torch.Tensor, pair_keep: torch.Tensor) -> Optional[torch.Tensor]:
    """Segment ids of ``pair_keep`` (a ``[B or 1, L, L]`` view of ``mask``,
    not expanded over the batch), cached per mask object and version.  The
    ids keep the mask's own batch extent; callers expand them."""
    version = tensor_version(mask)
    hit = _SEGMENTS_OF.get(mask) if version is not None else None
    if hit is not None and hit[0] == version:
        return hit[1]
    ids = dense_as_segments(pair_keep)
    if version is not None:
        _SEGMENTS_OF[mask] = (version, ids)
    return ids


# key mask -> (its version, event, pinned flag): whether every key is kept,
# found on the device without a host synchronisation.
_ALL_KEPT: WeakIdKeyDictionary = WeakIdKeyDictionary()


def _all_kept(mask: torch.Tensor, key_keep: torch.Tensor) -> bool:
    """True when ``key_keep`` (a ``[B or 1, K]`` byte view of ``mask``) keeps
    every key, as found by an earlier call with the same mask object and
    version.  The check runs on the device and is read back through pinned
    memory once its event has completed, so no call waits for the GPU: the
    first call with a mask starts the check and answers False, later calls
    answer True once the check has finished and found every key kept.  Such
    a mask then runs as no mask (the same results: every pair is kept and
    no row is dead), on the kernels without masking or launch order."""
    version = tensor_version(mask)
    if version is None:  # no version counter: no check can be reused
        return False
    hit = _ALL_KEPT.get(mask)
    if hit is not None and hit[0] == version:
        return hit[1].query() and bool(hit[2])
    flag = torch.zeros((), dtype=torch.bool, pin_memory=True)
    stream = torch.cuda.current_stream(key_keep.device)  # the copy's stream: the mask's device's
    with torch.cuda.stream(stream):
        flag.copy_(key_keep.bool().all(), non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
    _ALL_KEPT[mask] = (version, ev, flag)
    return False


def kernel_masks(
    attention_mask: "Optional[torch.Tensor | SegmentMask]",
    batch: int,
    query_len: int,
    key_len: int,
    device: Optional[torch.device] = None,
    segments_from_dense: bool = True,
    heads: Optional[int] = None,
) -> tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Split a rank-4 keep mask into the kernels' ``(key_keep, pair_keep)``.

    ``(B|1, 1, 1, K)`` becomes a ``[B, K]`` byte view (``key_keep``), or
    no mask once an asynchronous device check has found that it keeps every
    key (``_all_kept``),
    ``(B|1, 1, Q, K)`` a ``[B, Q, K]`` byte view (``pair_keep``), a per-head
    ``(B|1, H, Q|1, K)`` mask (``heads`` = H given) a ``[B, H, Q, K]`` one, or, for a
    dense mask of the packed-document form on the GPU in eager mode, the
    equivalent int32 segment ids (``dense_as_segments``; off with
    ``segments_from_dense=False``).  A batch
    dimension of 1 is broadcast with stride 0.  A ``SegmentMask`` becomes
    ``int32 [B, S]`` segment ids in the ``key_keep`` slot, on ``device``
    (default: the ids' own).  ``None`` means no mask.
    """
    if attention_mask is None:
        return None, None
    if isinstance(attention_mask, SegmentMask):
        ids = attention_mask.doc_ids
        if ids.shape[0] != batch or ids.shape[1] != key_len or query_len != key_len:
            raise ValueError(
                f"SegmentMask of shape {tuple(ids.shape)} does not match (B={batch}, Q={query_len}, K={key_len})"
            )
        return attention_mask.segment_ids(device if device is not None else ids.device), None
    keep = normalize_keep_mask(attention_mask)
    if keep.ndim != 4:
        raise ValueError(f"attention_mask must be rank-4 [B,1,Q,K]; got shape={tuple(keep.shape)}")
    if keep.shape[1] != 1 and (heads is None or keep.shape[1] != heads):
        raise ValueError(
            f"attention_mask head dim must be 1 or the number of heads ({heads}); got shape={tuple(keep.shape)}"
        )
    if keep.shape[0] not in (1, batch) or keep.shape[-1] != key_len or keep.shape[-2] not in (1, query_len):
        raise ValueError(
            f"attention_mask shape {tuple(keep.shape)} does not broadcast to (B={batch},1,Q={query_len},K={key_len})"
        )
    if query_len != key_len:
        raise ValueError("masked attention needs query_len == key_len (query liveness is read from the mask)")
    bytes_ = keep.view(torch.uint8) if keep.dtype == torch.bool else keep.to(torch.uint8)
    if keep.shape[1] != 1:
        return None, _per_head_pair_mask(bytes_, batch, heads, query_len, key_len)
    if keep.shape[-2] == 1:
        kk = bytes_[:, 0, 0, :]
        # a key mask that keeps every key runs as no mask (eager mode on the
        # GPU; the check never waits for the device)
        if (
            kk.is_cuda
            and not torch.compiler.is_compiling()
            and not torch.cuda.is_current_stream_capturing()
            and _all_kept(attention_mask, kk)
        ):
            return None, None
        if kk.stride(-1) != 1:
            kk = kk.contiguous()
        return kk.expand(batch, key_len), None
    pk = bytes_[:, 0, :, :]
    # A dense mask of the packed-document form runs as segment ids (the
    # kernels then skip the tiles between documents); checked once per mask
    # tensor and version, in eager mode on the GPU only.
    if segments_from_dense and pk.is_cuda and not torch.compiler.is_compiling():
        ids = _segments_cached(attention_mask, pk)
        if ids is not None:
            ids = ids.to(device) if device is not None else ids
            # a broadcast (1, 1, S, S) mask gives one row of ids, read with
            # batch stride 0
            return ids.expand(batch, key_len), None
    # the kernels read 16-byte chunks of the rows: rows 16-byte aligned,
    # row and batch strides multiples of 16 bytes, each row's allocation
    # reaching the next multiple of 16 past key_len (zero padding)
    k16 = (key_len + 15) // 16 * 16
    if (
        pk.stride(-1) != 1
        or pk.data_ptr() % 16
        or pk.stride(-2) % 16
        or pk.stride(-2) < k16
        or (pk.shape[0] > 1 and pk.stride(0) % 16)
    ):
        padded = torch.zeros(pk.shape[0], pk.shape[1], k16, dtype=torch.uint8, device=pk.device)
        padded[:, :, :key_len] = pk
        pk = padded[:, :, :key_len]
    return None, pk.expand(batch, query_len, key_len)


def _per_head_pair_mask(bytes_: torch.Tensor, batch: int, heads: int, query_len: int, key_len: int) -> torch.Tensor:
    """``[B, H, Q, K]`` byte view of a per-head ``(B|1, H, Q|1, K)`` keep mask
    in the layout the kernels read (rows in 16-byte chunks: 16-byte aligned,
    row, head and batch strides multiples of 16 bytes, each row's allocation
    reaching the next multiple of 16 past ``key_len``); copied into a
    padded buffer when the view does not qualify."""
    k16 = (key_len + 15) // 16 * 16
    pk = bytes_
    if pk.shape[-2] == 1:  # per-head key padding: one row per head, read for every query
        pk = pk.expand(pk.shape[0], heads, query_len, key_len)
    ok = (
        pk.stride(-1) == 1
        and pk.data_ptr() % 16 == 0
        and (pk.stride(-2) % 16 == 0 and pk.stride(-2) >= k16 or pk.stride(-2) == 0 and key_len % 16 == 0)
        and pk.stride(1) % 16 == 0
        and (pk.shape[0] == 1 or pk.stride(0) % 16 == 0)
    )
    if not ok:
        padded = torch.zeros(pk.shape[0], heads, query_len, k16, dtype=torch.uint8, device=pk.device)
        padded[..., :key_len] = pk
        pk = padded[..., :key_len]
    return pk.expand(batch, heads, query_len, key_len)
