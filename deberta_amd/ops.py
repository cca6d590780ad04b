"""torch.library custom ops over the HIP kernels of ``libdsa.so``.

``deberta_amd::dsa_fwd`` and ``deberta_amd::dsa_bwd`` are functional (they
allocate their outputs and mutate nothing), carry fake-tensor
implementations for ``torch.compile``, and are linked by
``register_autograd``.  They have a CUDA/HIP implementation only: called on
CPU tensors they raise, there is no fallback.

Tensor layouts (see include/dsa.h):
  q, k, v           [B, L, H, D] views, head dim contiguous
  kr, qr            [H, 2A, D] views (projected relative tables) or None
  rel_table         int32 [Lq + Lk - 1]: relative position of offset i - j at
                    index (i - j) + (Lk - 1)
  key_keep          uint8 [B, Lk] (broadcast keep mask), or int32 [B, L]
                    segment ids (0: inactive token; pair (i, j) kept iff
                    both ids are equal and nonzero), or None
  pair_keep         uint8 [B, Lq, Lk] or [B, H, Lq, Lk] (per-head) or None
                    (pairwise keep mask)
  out               [B, Lq, H, D] contiguous, dtype of q
  lse               float32 [B, H, Lq]
  bias              [B, H, pad128(Lq), pad128(Lk)] the relative score term
                    c2p + p2c saved for the backward (float16 for bfloat16
                    inputs, float32 for float32); empty when not saved
  qc                [B, Lq, H, D] or None: the query rows of the c2p term
                    (q when None); the p2p term rides on it (attention.py)
  dropout_t         attention dropout threshold in [0, 65535]: each
                    probability is dropped with probability t / 65536, the
                    kept ones scaled by 65536 / (65536 - t); 0: no dropout
  dropout_seed      int64 CPU tensor of one element (or None without
                    dropout): the 64-bit seed of the keep bits
  drop_bits         uint8 [aux_bytes]: what the forward leaves for the
                    backward besides bias: the keep bits dsa_fwd generated
                    (dropout_bytes; none without dropout), then, for bfloat16
                    with the relative term saved and sequences longer than
                    2 att_span, O's rounding residual (dsa_fwd_args.out_lo,
                    bfloat16 [B, Lq, H, D] at a 256-byte aligned offset);
                    empty when there is neither
"""

from __future__ import annotations

import ctypes
import warnings
from typing import Optional

import torch
from torch import Tensor

from deberta_amd import _eager, _lib

_DTYPES = {torch.float32: _lib.DSA_F32, torch.bfloat16: _lib.DSA_BF16}


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _strides3(t: Tensor) -> tuple[int, int, int]:
    s = t.stride()
    return (s[0], s[1], s[2])


def _vec(dtype: torch.dtype) -> int:
    return 16 // (2 if dtype == torch.bfloat16 else 4)


def _kernel_ready(t: Tensor) -> Tensor:
    """Return ``t`` if the kernels can read it in place (head dim contiguous,
    16-byte aligned rows), else a contiguous copy."""
    vec = _vec(t.dtype)
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % vec == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def _flags(kr: Optional[Tensor], qr: Optional[Tensor]) -> int:
    return (_lib.DSA_C2P if kr is not None else 0) | (_lib.DSA_P2C if qr is not None else 0)


def _pad128(n: int) -> int:
    return (n + 127) // 128 * 128


def bias_shape(q: Tensor, k: Tensor) -> tuple[int, int, int, int]:
    """Shape of the saved relative term (``dsa_fwd_args.bias``)."""
    return (q.shape[0], q.shape[2], _pad128(q.shape[1]), _pad128(k.shape[1]))


def bias_dtype(dtype: torch.dtype) -> torch.dtype:
    return torch.float16 if dtype == torch.bfloat16 else torch.float32


def dropout_bytes(q: Tensor, k: Tensor, dropout_t: int) -> int:
    """Bytes of the keep bits (``dsa_fwd_dropout_bytes``): one 32-bit word
    per (b, h, 32 queries, 64 keys, lane) of the padded extents."""
    if not dropout_t:
        return 0
    B, Lq, H = q.shape[0], q.shape[1], q.shape[2]
    return B * H * (_pad128(Lq) // 32) * (_pad128(k.shape[1]) // 64) * 64 * 4


def dropout_threshold(p: float) -> int:
    """The kernels' dropout threshold for probability ``p``: ``round(p *
    65536)``.  The kernels drop with probability ``t / 65536`` exactly, so a
    ``p`` whose threshold is 0 or 65536 (``p < 2^-17`` or ``p > 1 - 2^-17``)
    has no kernel form; the module runs those on its torch path."""
    return int(round(float(p) * 65536.0))


def draw_dropout_seed() -> Tensor:
    """A fresh 62-bit seed for the keep bits, drawn from torch's default CPU
    generator (so ``torch.manual_seed`` reproduces it, and activation
    checkpointing, which restores the RNG states, redraws the same one)."""
    return torch.randint(0, 1 << 62, (1,), dtype=torch.int64)


def _seed_value(seed: Optional[Tensor], t: int) -> int:
    if not t:
        return 0
    if seed is None or seed.numel() != 1 or seed.dtype != torch.int64 or seed.device.type != "cpu":
        raise ValueError("dsa: dropout needs dropout_seed, an int64 CPU tensor of one element")
    return int(seed.reshape(()).item()) & 0xFFFFFFFFFFFFFFFF


def residual_wanted(q: Tensor, k: Tensor, relative: bool, att_span: int, save_bias: bool) -> bool:
    """Whether the forward writes O's rounding residual for the backward's
    row sums dO . O (``dsa_fwd_args.out_lo``): bfloat16, the relative term
    saved (a backward will follow) and a sequence longer than 2 att_span,
    where the table rows aggregate several offsets each and a row sum of
    dKr / dQr can keep the per-row offset that a bf16-rounded O puts into
    dS.  Up to that length (the benchmarked shape included) nothing is
    written."""
    return q.dtype == torch.bfloat16 and relative and save_bias and max(q.shape[1], k.shape[1]) > 2 * int(att_span)


def aux_layout(q: Tensor, k: Tensor, dropout_t: int, residual: bool) -> tuple[int, int, int]:
    """(keep-bit bytes, byte offset of O's residual, total bytes) of the
    forward's fourth output."""
    nd = dropout_bytes(q, k, dropout_t)
    if not residual:
        return nd, nd, nd
    off = (nd + 255) // 256 * 256
    return nd, off, off + q.shape[0] * q.shape[1] * q.shape[2] * q.shape[3] * 2


def _check_threshold(t: int) -> None:
    if not 0 <= int(t) <= 65535:
        raise ValueError(f"dsa: dropout threshold must be in [0, 65535] (units of 1/65536), got {t}")


def _fill_fwd_args(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    out: Tensor,
    lse: Tensor,
    att_span: int,
    scale: float,
    bias: Optional[Tensor] = None,
    qc: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
    dropout_bits: Optional[Tensor] = None,
) -> _lib.DsaFwdArgs:
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    a = _lib.DsaFwdArgs()
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.kr, a.qr = _ptr(kr), _ptr(qr)
    a.rel_table = _ptr(rel_table)
    if key_keep is not None and key_keep.dtype == torch.int32:
        a.seg, a.seg_stride_b = key_keep.data_ptr(), key_keep.stride(0)
        key_keep = None
    a.key_keep, a.pair_keep = _ptr(key_keep), _ptr(pair_keep)
    a.out, a.lse = out.data_ptr(), lse.data_ptr()
    a.bias = _ptr(bias) if bias is not None and bias.numel() else None
    a.q_strides[:] = _strides3(q)
    a.k_strides[:] = _strides3(k)
    a.v_strides[:] = _strides3(v)
    a.o_strides[:] = _strides3(out)
    if kr is not None:
        a.kr_strides[:] = (kr.stride(0), kr.stride(1))
    if qr is not None:
        a.qr_strides[:] = (qr.stride(0), qr.stride(1))
    if key_keep is not None:
        a.key_keep_stride_b = key_keep.stride(0)
    if pair_keep is not None:
        if pair_keep.dim() == 4:  # per head: [B, H, Lq, Lk]
            a.pair_keep_strides[:] = (pair_keep.stride(0), pair_keep.stride(2))
            a.pair_keep_stride_h = pair_keep.stride(1)
        else:
            a.pair_keep_strides[:] = (pair_keep.stride(0), pair_keep.stride(1))
    a.B, a.H, a.Lq, a.Lk, a.D = B, H, Lq, Lk, D
    a.att_span = int(att_span)
    a.dtype = _DTYPES[q.dtype]
    a.flags = _flags(kr, qr)
    a.scale = float(scale)
    if qc is not None:
        a.qc = qc.data_ptr()
        a.qc_strides[:] = _strides3(qc)
    _check_threshold(dropout_t)
    a.dropout_threshold = int(dropout_t)
    a.dropout_seed = _seed_value(dropout_seed, int(dropout_t))
    if dropout_bits is not None and dropout_bits.numel():
        # the forward's fourth output: keep bits, then O's residual
        residual = residual_wanted(q, k, a.flags != 0, att_span, a.bias is not None)
        nd, lo_off, total = aux_layout(q, k, dropout_t, residual)
        if dropout_bits.numel() * dropout_bits.element_size() < total:
            raise ValueError("dsa: dropout_bits is smaller than the call's keep bits and O's residual")
        if dropout_t and nd:
            a.dropout_bits = dropout_bits.data_ptr()
        if residual:
            if not (out.is_contiguous() and out.dtype == torch.bfloat16):
                raise ValueError("dsa: O's residual needs a contiguous bfloat16 out")
            a.out_lo = dropout_bits.data_ptr() + lo_off
    return a


def _validate(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    att_span: int,
    qc: Optional[Tensor] = None,
) -> None:
    if q.dtype not in _DTYPES:
        raise TypeError(f"dsa: q dtype must be float32 or bfloat16, got {q.dtype}")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("dsa: q, k, v must be [B, L, H, D]")
    B, Lq, H, D = q.shape
    if k.shape[0] != B or k.shape[2:] != (H, D) or v.shape != k.shape:
        raise ValueError(f"dsa: shape mismatch q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if D not in (32, 64):
        raise ValueError(f"dsa: head dim must be 32 or 64, got {D}")
    for name, t in (("k", k), ("v", v), ("kr", kr), ("qr", qr)):
        if t is not None and t.dtype != q.dtype:
            raise TypeError(f"dsa: {name} dtype {t.dtype} differs from q dtype {q.dtype}")
    R = 2 * int(att_span)
    for name, t in (("kr", kr), ("qr", qr)):
        if t is not None and (t.dim() != 3 or t.shape[0] != H or t.shape[1] != R or t.shape[2] != D):
            raise ValueError(f"dsa: {name} must be [H={H}, 2A={R}, D={D}], got {tuple(t.shape)}")
    if (kr is not None or qr is not None) and (rel_table is None or rel_table.numel() != Lq + k.shape[1] - 1):
        raise ValueError("dsa: rel_table of Lq + Lk - 1 entries is required with relative tables")
    if key_keep is not None and pair_keep is not None:
        raise ValueError("dsa: give at most one of key_keep and pair_keep")
    # The kernels index the masks by (b, i) / (b, i, j) over the full batch:
    # a mask of another extent would be read out of bounds.
    Lk = k.shape[1]
    if key_keep is not None:
        if key_keep.dtype not in (torch.uint8, torch.int32):
            raise TypeError(f"dsa: key_keep must be uint8 (keep bytes) or int32 (segment ids), got {key_keep.dtype}")
        if key_keep.dim() != 2 or tuple(key_keep.shape) != (B, Lk) or key_keep.stride(-1) != 1:
            raise ValueError(f"dsa: key_keep / segment ids must be [B={B}, Lk={Lk}] with unit key stride, "
                             f"got {tuple(key_keep.shape)} strides {key_keep.stride()}")
        if key_keep.device != q.device:
            raise ValueError("dsa: key_keep must be on q's device")
    if pair_keep is not None:
        if pair_keep.dtype != torch.uint8:
            raise TypeError(f"dsa: pair_keep must be uint8, got {pair_keep.dtype}")
        shapes = ((B, Lq, Lk), (B, H, Lq, Lk))
        if tuple(pair_keep.shape) not in shapes or pair_keep.stride(-1) != 1:
            raise ValueError(f"dsa: pair_keep must be [B={B}, Lq={Lq}, Lk={Lk}] or [B, H={H}, Lq, Lk] with unit "
                             f"key stride, got {tuple(pair_keep.shape)} strides {pair_keep.stride()}")
        if pair_keep.device != q.device:
            raise ValueError("dsa: pair_keep must be on q's device")
    if qc is not None:
        if kr is None:
            raise ValueError("dsa: qc (the c2p term's query rows) needs the pos-key table kr")
        if qc.shape != q.shape or qc.dtype != q.dtype:
            raise ValueError(f"dsa: qc must match q ({tuple(q.shape)}, {q.dtype}), got {tuple(qc.shape)}, {qc.dtype}")


def _dsa_fwd_impl(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    att_span: int,
    scale: float,
    save_bias: bool = True,
    qc: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(out, lse, bias, drop_bits).  With c2p/p2c and ``save_bias`` the
    relative score term is written to ``bias`` for the backward (which
    needs it); else ``bias`` is empty.  ``qc``: the c2p term's query rows (q
    when None).  ``dropout_t`` / ``dropout_seed``: attention dropout (lse is
    that of the probabilities before dropout); its keep bits come back in
    ``drop_bits`` for the backward, followed by O's rounding residual when
    ``residual_wanted`` (empty when there is neither)."""
    _eager.refuse_capture("deberta_amd::dsa_fwd")
    _validate(q, k, v, kr, qr, rel_table, key_keep, pair_keep, att_span, qc)
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    kr = None if kr is None else _kernel_ready(kr)
    qr = None if qr is None else _kernel_ready(qr)
    qc = None if qc is None else _kernel_ready(qc)
    B, Lq, H, D = q.shape
    out = torch.empty((B, Lq, H, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, Lq), dtype=torch.float32, device=q.device)
    if save_bias and (kr is not None or qr is not None):
        bias = torch.empty(bias_shape(q, k), dtype=bias_dtype(q.dtype), device=q.device)
    else:
        bias = torch.empty((0,), dtype=bias_dtype(q.dtype), device=q.device)
    residual = residual_wanted(q, k, kr is not None or qr is not None, att_span, save_bias)
    drop_bits = torch.empty((aux_layout(q, k, dropout_t, residual)[2],), dtype=torch.uint8, device=q.device)
    args = _fill_fwd_args(
        q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, att_span, scale, bias, qc, dropout_t, dropout_seed,
        drop_bits,
    )
    lib = _lib.load()
    # scratch for the heaviest-first launch order under key / segment masks,
    # the table copies and dropout's keep bits
    nws = lib.dsa_fwd_workspace_bytes(ctypes.byref(args))
    ws = torch.empty((nws,), dtype=torch.uint8, device=q.device) if nws else None
    if ws is not None:
        args.workspace, args.workspace_bytes = ws.data_ptr(), nws
    _lib.check(lib.dsa_fwd(ctypes.byref(args), ctypes.c_void_p(_eager.stream_ptr(q))), "dsa_fwd")
    return out, lse, bias, drop_bits


# Tagged CUDA-graph unsafe: capturing the op's forward and backward in a HIP
# graph ended in a host fault inside the runtime's capture end, whose cause is
# not known.  Under torch.compile's CUDA-graph modes (reduce-overhead,
# max-autotune) inductor then runs these ops outside the captured graphs
# (graph partitions around them) instead of capturing them.
_TAGS = (torch.Tag.cudagraph_unsafe,)

dsa_fwd = torch.library.custom_op(
    "deberta_amd::dsa_fwd", _dsa_fwd_impl, mutates_args=(), device_types="cuda", tags=_TAGS
)


@dsa_fwd.register_fake
def _dsa_fwd_fake(
    q, k, v, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias=True, qc=None, dropout_t=0,
    dropout_seed=None,
):
    B, Lq, H, D = q.shape
    out = q.new_empty((B, Lq, H, D))
    lse = q.new_empty((B, H, Lq), dtype=torch.float32)
    if save_bias and (kr is not None or qr is not None):
        bias = q.new_empty(bias_shape(q, k), dtype=bias_dtype(q.dtype))
    else:
        bias = q.new_empty((0,), dtype=bias_dtype(q.dtype))
    residual = residual_wanted(q, k, kr is not None or qr is not None, att_span, save_bias)
    return out, lse, bias, q.new_empty((aux_layout(q, k, dropout_t, residual)[2],), dtype=torch.uint8)


def bwd_workspace_bytes(args: _lib.DsaBwdArgs) -> int:
    return int(_lib.load().dsa_bwd_workspace_bytes(ctypes.byref(args)))


def fill_bwd_args(
    dout: Tensor,
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    out: Tensor,
    lse: Tensor,
    bias: Optional[Tensor],
    att_span: int,
    scale: float,
    dq: Tensor,
    dk: Tensor,
    dv: Tensor,
    dkr: Optional[Tensor],
    dqr: Optional[Tensor],
    dtab_overwrite: bool = False,
    qc: Optional[Tensor] = None,
    dqc: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
    dropout_bits: Optional[Tensor] = None,
) -> _lib.DsaBwdArgs:
    """Backward arguments.  dkr / dqr are fp32 and accumulated into, or, with
    ``dtab_overwrite``, written (fp32 or bf16, their dtype).  With ``qc``,
    ``dqc`` receives its gradient (the c2p part of dq).  The dropout
    arguments are the forward's (with its keep bits, none are generated;
    without, they are regenerated from the seed)."""
    a = _lib.DsaBwdArgs()
    a.fwd = _fill_fwd_args(
        q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, att_span, scale, bias, qc, dropout_t, dropout_seed,
        dropout_bits,
    )
    if dqc is not None:
        a.dqc = dqc.data_ptr()
        a.dqc_strides[:] = _strides3(dqc)
    a.dout = dout.data_ptr()
    a.do_strides[:] = _strides3(dout)
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    a.dq_strides[:] = _strides3(dq)
    a.dk_strides[:] = _strides3(dk)
    a.dv_strides[:] = _strides3(dv)
    a.dkr, a.dqr = _ptr(dkr), _ptr(dqr)
    a.stages = 0
    tab = dkr if dkr is not None else dqr
    a.dtab_dtype = _DTYPES[tab.dtype] if tab is not None else _lib.DSA_F32
    a.dtab_overwrite = int(dtab_overwrite)
    return a


def _alert_nondeterministic_tables() -> None:
    """torch's deterministic-algorithms contract: the relative-table
    gradients are summed with fp32 atomics, so their last bits vary from run
    to run (every other output is bitwise reproducible).  Raises under
    ``torch.use_deterministic_algorithms(True)``, warns under
    ``warn_only=True``."""
    if not torch.are_deterministic_algorithms_enabled():
        return
    msg = (
        "deberta_amd::dsa_bwd does not have a deterministic implementation of the relative-table "
        "gradients (dkr / dqr are accumulated with fp32 atomics), but you set "
        "'torch.use_deterministic_algorithms(True)'."
    )
    if torch.is_deterministic_algorithms_warn_only_enabled():
        warnings.warn(msg)
    else:
        raise RuntimeError(msg)


def _dsa_bwd_impl(
    dout: Tensor,
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    out: Tensor,
    lse: Tensor,
    bias: Tensor,
    att_span: int,
    scale: float,
    qc: Optional[Tensor] = None,
    dqkv: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
    drop_bits: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients (dq, dk, dv, dkr, dqr, dqc).  With ``dqkv`` (a contiguous
    ``[B, L, 3, H, D]`` buffer), dq, dk and dv are written into its three
    slices and returned as views of it.  dkr/dqr are [H, 2A, D] in the
    tables' dtype (empty when the matching table is None).  ``bias`` is the
    relative term dsa_fwd saved (required with c2p/p2c).  With ``qc`` (the
    c2p term's query rows), dqc is its gradient and dq the content part;
    else dqc is empty.  ``dropout_t`` / ``dropout_seed`` / ``drop_bits``:
    the forward's (without its keep bits the kernels regenerate them)."""
    _eager.refuse_capture("deberta_amd::dsa_bwd")
    if kr is not None or qr is not None:
        _alert_nondeterministic_tables()
    q, k, v = _kernel_ready(q), _kernel_ready(k), _kernel_ready(v)
    kr = None if kr is None else _kernel_ready(kr)
    qr = None if qr is None else _kernel_ready(qr)
    qc = None if qc is None else _kernel_ready(qc)
    if (kr is not None or qr is not None) and tuple(bias.shape) != bias_shape(q, k):
        raise RuntimeError("dsa_bwd: the relative term saved by dsa_fwd (save_bias=True) is required")
    dout = _kernel_ready(dout.to(q.dtype))
    out = _kernel_ready(out)
    B, Lq, H, D = q.shape
    R = 2 * int(att_span)
    if dqkv is not None:  # the three gradients as slices of one packed buffer
        dq, dk, dv = dqkv.unbind(2)
    else:
        dq = torch.empty_like(q, memory_format=torch.contiguous_format)
        dk = torch.empty_like(k, memory_format=torch.contiguous_format)
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    # the table gradients are written in the tables' dtype (no zeroing, no cast)
    tab = dict(dtype=q.dtype, device=q.device)
    dkr = torch.empty((H, R, D), **tab) if kr is not None else torch.empty((0,), **tab)
    dqr = torch.empty((H, R, D), **tab) if qr is not None else torch.empty((0,), **tab)
    dqc = torch.empty_like(q, memory_format=torch.contiguous_format) if qc is not None else torch.empty((0,), **tab)
    args = fill_bwd_args(
        dout, q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, att_span, scale,
        dq, dk, dv, dkr if kr is not None else None, dqr if qr is not None else None, dtab_overwrite=True,
        qc=qc, dqc=dqc if qc is not None else None, dropout_t=dropout_t, dropout_seed=dropout_seed,
        dropout_bits=drop_bits,
    )
    ws = torch.empty((max(bwd_workspace_bytes(args), 16),), dtype=torch.uint8, device=q.device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = ws.numel()
    lib = _lib.load()
    _lib.check(lib.dsa_bwd(ctypes.byref(args), ctypes.c_void_p(_eager.stream_ptr(q))), "dsa_bwd")
    return dq, dk, dv, dkr, dqr, dqc


dsa_bwd = torch.library.custom_op(
    "deberta_amd::dsa_bwd", _dsa_bwd_impl, mutates_args=(), device_types="cuda", tags=_TAGS
)


@dsa_bwd.register_fake
def _dsa_bwd_fake(
    dout, q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, att_span, scale, qc=None, dqkv=None,
    dropout_t=0, dropout_seed=None, drop_bits=None,
):
    H, D = q.shape[2], q.shape[3]
    R = 2 * int(att_span)
    dkr = q.new_empty((H, R, D)) if kr is not None else q.new_empty((0,))
    dqr = q.new_empty((H, R, D)) if qr is not None else q.new_empty((0,))
    dqc = q.new_empty(q.shape) if qc is not None else q.new_empty((0,))
    return (
        q.new_empty(q.shape),
        k.new_empty(k.shape),
        v.new_empty(v.shape),
        dkr,
        dqr,
        dqc,
    )


def _setup_context(ctx, inputs, output):
    q, k, v, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed = (
        _with_dropout(inputs, 12)
    )
    out, lse, bias, drop_bits = output
    ctx.mark_non_differentiable(lse, bias, drop_bits)
    # lse, the saved term and the keep bits get no gradient: do not
    # materialise zeros for them (the saved term is (B, H, L, L)-sized)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, qc, dropout_seed, drop_bits)
    ctx.att_span = att_span
    ctx.scale = scale
    ctx.dropout_t = dropout_t


def _with_dropout(inputs: tuple, n: int) -> tuple:
    """The op's inputs with the two trailing dropout arguments filled in
    (callers may leave them out)."""
    return tuple(inputs) + (0, None)[len(inputs) - n:] if len(inputs) < n + 2 else tuple(inputs)


def _backward(ctx, dout, dlse, dbias, ddrop):
    q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, qc, dropout_seed, drop_bits = ctx.saved_tensors
    if dout is None:  # the output itself received no gradient
        return (None,) * 14
    dq, dk, dv, dkr, dqr, dqc = _eager.on_eager(ctx, dsa_bwd, _dsa_bwd_impl)(
        dout, q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, ctx.att_span, ctx.scale, qc, None,
        ctx.dropout_t, dropout_seed, drop_bits,
    )
    return (
        dq, dk, dv, (dkr if kr is not None else None), (dqr if qr is not None else None),
        None, None, None, None, None, None, (dqc if qc is not None else None), None, None,
    )


torch.library.register_autograd("deberta_amd::dsa_fwd", _backward, setup_context=_setup_context)
_DsaFwdFunction = _eager.function("_DsaFwdFunction", _dsa_fwd_impl, _setup_context, _backward)


def attention(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    att_span: int,
    scale: float,
    save_bias: bool = True,
    qc: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``deberta_amd::dsa_fwd`` with its autograd: the op itself under
    torch.compile or tracing, its implementation in a torch.autograd.Function
    in plain eager mode (the same kernels, less host time)."""
    if _eager.eager(q):
        return _DsaFwdFunction.apply(
            q, k, v, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed
        )
    return torch.ops.deberta_amd.dsa_fwd(
        q, k, v, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed
    )


# ---- packed q, k, v ----------------------------------------------------------------
# The module's q, k and v are slices of one fused projection, (B, L, 3, H, D).
# Given that tensor itself, the op's backward writes dq, dk and dv into one
# buffer of the same layout and returns it as the projection's gradient: no
# stack of three gradients and no copy.


def _dsa_fwd_packed_impl(
    qkv: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    att_span: int,
    scale: float,
    save_bias: bool = True,
    qc: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``dsa_fwd`` on ``q, k, v = qkv.unbind(2)`` (qkv ``[B, L, 3, H, D]``)."""
    if qkv.dim() != 5 or qkv.shape[2] != 3:
        raise ValueError(f"dsa: qkv must be [B, L, 3, H, D], got {tuple(qkv.shape)}")
    q, k, v = qkv.unbind(2)
    return _dsa_fwd_impl(
        q, k, v, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed
    )


dsa_fwd_packed = torch.library.custom_op(
    "deberta_amd::dsa_fwd_packed", _dsa_fwd_packed_impl, mutates_args=(), device_types="cuda", tags=_TAGS
)


@dsa_fwd_packed.register_fake
def _dsa_fwd_packed_fake(
    qkv, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias=True, qc=None, dropout_t=0,
    dropout_seed=None,
):
    q, k, _ = qkv.unbind(2)
    return _dsa_fwd_fake(
        q, k, k, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed
    )


def _dsa_bwd_packed_impl(
    dout: Tensor,
    qkv: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    out: Tensor,
    lse: Tensor,
    bias: Tensor,
    att_span: int,
    scale: float,
    qc: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
    drop_bits: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients (dqkv, dkr, dqr, dqc) of ``dsa_fwd_packed``: dqkv a
    contiguous ``[B, L, 3, H, D]`` tensor in qkv's dtype."""
    q, k, v = qkv.unbind(2)
    dqkv = torch.empty(qkv.shape, dtype=qkv.dtype, device=qkv.device)
    _, _, _, dkr, dqr, dqc = _dsa_bwd_impl(
        dout, q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, att_span, scale, qc, dqkv=dqkv,
        dropout_t=dropout_t, dropout_seed=dropout_seed, drop_bits=drop_bits,
    )
    return dqkv, dkr, dqr, dqc


dsa_bwd_packed = torch.library.custom_op(
    "deberta_amd::dsa_bwd_packed", _dsa_bwd_packed_impl, mutates_args=(), device_types="cuda", tags=_TAGS
)


@dsa_bwd_packed.register_fake
def _dsa_bwd_packed_fake(
    dout, qkv, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, att_span, scale, qc=None, dropout_t=0,
    dropout_seed=None, drop_bits=None,
):
    q, k, v = qkv.unbind(2)
    _, _, _, dkr, dqr, dqc = _dsa_bwd_fake(
        dout, q, k, v, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, att_span, scale, qc
    )
    return qkv.new_empty(qkv.shape), dkr, dqr, dqc


def _setup_context_packed(ctx, inputs, output):
    qkv, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed = (
        _with_dropout(inputs, 10)
    )
    out, lse, bias, drop_bits = output
    ctx.mark_non_differentiable(lse, bias, drop_bits)
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(qkv, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, qc, dropout_seed, drop_bits)
    ctx.att_span = att_span
    ctx.scale = scale
    ctx.dropout_t = dropout_t


def _backward_packed(ctx, dout, dlse, dbias, ddrop):
    qkv, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, qc, dropout_seed, drop_bits = ctx.saved_tensors
    if dout is None:
        return (None,) * 12
    dqkv, dkr, dqr, dqc = _eager.on_eager(ctx, dsa_bwd_packed, _dsa_bwd_packed_impl)(
        dout, qkv, kr, qr, rel_table, key_keep, pair_keep, out, lse, bias, ctx.att_span, ctx.scale, qc,
        ctx.dropout_t, dropout_seed, drop_bits,
    )
    return (
        dqkv, (dkr if kr is not None else None), (dqr if qr is not None else None),
        None, None, None, None, None, None, (dqc if qc is not None else None), None, None,
    )


torch.library.register_autograd("deberta_amd::dsa_fwd_packed", _backward_packed, setup_context=_setup_context_packed)
_DsaFwdPackedFunction = _eager.function("_DsaFwdPackedFunction", _dsa_fwd_packed_impl, _setup_context_packed, _backward_packed)


def attention_packed(
    qkv: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    key_keep: Optional[Tensor],
    pair_keep: Optional[Tensor],
    att_span: int,
    scale: float,
    save_bias: bool = True,
    qc: Optional[Tensor] = None,
    dropout_t: int = 0,
    dropout_seed: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """``attention`` on packed ``qkv`` ``[B, L, 3, H, D]``: the gradient of
    qkv comes back as one tensor."""
    if _eager.eager(qkv):
        return _DsaFwdPackedFunction.apply(
            qkv, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed
        )
    return torch.ops.deberta_amd.dsa_fwd_packed(
        qkv, kr, qr, rel_table, key_keep, pair_keep, att_span, scale, save_bias, qc, dropout_t, dropout_seed
    )


def _dsa_bias_impl(
    q: Tensor,
    k: Tensor,
    kr: Optional[Tensor],
    qr: Optional[Tensor],
    rel_table: Optional[Tensor],
    att_span: int,
    scale: float,
    qc: Optional[Tensor] = None,
) -> Tensor:
    """The relative score term ``scale * (c2p + p2c)`` as ``(B, H, Lq, Lk)``
    in q's dtype (the reference's ``disentangled_attention_bias``,
    deberta_v2_native.py:530-562), unmasked; zeros without tables.  q, k are
    ``[B, L, H, D]`` views; ``qc`` the c2p term's query rows (q when None)."""
    _eager.refuse_capture("deberta_amd::dsa_bias")
    _validate(q, k, k, kr, qr, rel_table, None, None, att_span, qc)
    q, k = _kernel_ready(q), _kernel_ready(k)
    kr = None if kr is None else _kernel_ready(kr)
    qr = None if qr is None else _kernel_ready(qr)
    qc = None if qc is None else _kernel_ready(qc)
    B, Lq, H, _ = q.shape
    Lk = k.shape[1]
    out = torch.empty((B, H, Lq, Lk), dtype=q.dtype, device=q.device)
    dummy = torch.empty((0,), dtype=torch.float32, device=q.device)
    args = _fill_fwd_args(q, k, k, kr, qr, rel_table, None, None, q, dummy, att_span, scale, None, qc)
    strides = (ctypes.c_int64 * 3)(*out.stride()[:3])
    lib = _lib.load()
    stream = _eager.stream_ptr(q)
    _lib.check(lib.dsa_bias(ctypes.byref(args), ctypes.c_void_p(out.data_ptr()), strides, ctypes.c_void_p(stream)), "dsa_bias")
    return out


dsa_bias = torch.library.custom_op(
    "deberta_amd::dsa_bias", _dsa_bias_impl, mutates_args=(), device_types="cuda", tags=_TAGS
)


@dsa_bias.register_fake
def _dsa_bias_fake(q, k, kr, qr, rel_table, att_span, scale, qc=None):
    B, Lq, H, _ = q.shape
    return q.new_empty((B, H, Lq, k.shape[1]))
