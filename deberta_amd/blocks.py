"""The blocks on either side of the attention, on the fused row kernels of
libdsa.so (include/dsa_block.h): the callers the reference runs right before
and after ``DisentangledSelfAttention``.

  FusedSelfOutput / FusedOutput   DebertaV2SelfOutput / DebertaV2Output
                                  (deberta_v2_native.py:115-165, 733-758):
                                  dense (a GEMM without its bias), then
                                  bias + residual + LayerNorm in one kernel
  FusedIntermediate               DebertaV2Intermediate (:703-730, "gelu"):
                                  dense, then bias + GELU in one kernel
  FusedRTDHead                    RTDHead (rtd.py:550-626): LayerNorm of
                                  hidden + the CLS context in one kernel,
                                  dense + bias + GELU, and the classifier
                                  fused with the discriminator's BCE loss
                                  (rtd.py:1134-1139) in ``forward_loss``
  RelativeEmbeddings              the encoder's shared relative-embedding
                                  table and its LayerNorm (get_rel_embedding,
                                  :1036-1047)

Parameter names are the reference's, so state dicts load unchanged.  The
GEMMs stay plain library GEMMs (hipBLASLt); everything between them runs in
the HIP kernels through the ``torch.library`` ops below, which have fake
implementations for ``torch.compile`` and autograd registrations.  Hidden
dropout p > 0 in training runs torch's dropout on the dense output (bias
included, as the reference's ``dropout(dense(x))``) and then the residual
LayerNorm kernel.  CPU tensors run the reference's blocks in torch
operations (the kernels run on the GPU only).
"""

from __future__ import annotations

import ctypes
from typing import Any, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from deberta_amd import _eager, _lib

# As the attention ops (deberta_amd/ops.py): under torch.compile's CUDA-graph
# modes these run between the captured graph partitions, not inside them
# (capturing the library's launches in a HIP graph ended in a host fault
# whose cause is not known).
_TAGS = (torch.Tag.cudagraph_unsafe,)

_DT = {torch.float32: _lib.DSA_F32, torch.bfloat16: _lib.DSA_BF16}


def _dt(t: Tensor, what: str) -> int:
    if t.dtype not in _DT:
        raise TypeError(f"{what}: dtype must be float32 or bfloat16, got {t.dtype}")
    return _DT[t.dtype]


def _rows(t: Tensor) -> Tensor:
    """``t`` as ``[N, C]`` rows with unit column stride (a view when possible)."""
    t2 = t.reshape(-1, t.shape[-1])
    if t2.stride(-1) != 1 or t2.stride(0) % 4 or t2.data_ptr() % (4 * t2.element_size()):
        t2 = t2.contiguous()
    return t2


def _stream(t: Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(_eager.stream_ptr(t))


def _ptr(t: Optional[Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _vec(t: Optional[Tensor]) -> Optional[Tensor]:
    return None if t is None else t.contiguous()


# ---------------------------------------------------------------------------
# add + LayerNorm


def _res_layout(res: Tensor, x: Tensor) -> tuple[Tensor, int, int, int]:
    """(tensor, group stride, row stride, rows per group) of a residual of
    x's shape: ``(N, C)``, or ``(B, S, C)`` possibly broadcast along S (the
    RTD head's CLS context, stride 0)."""
    if res.shape != x.shape:
        raise ValueError(f"add_ln: res must have x's shape {tuple(x.shape)}, got {tuple(res.shape)}")
    if res.stride(-1) != 1 or res.data_ptr() % (4 * res.element_size()):
        res = res.contiguous()
    if res.dim() == 2:
        return res, 0, res.stride(0), res.shape[0]
    if res.dim() == 3:
        if res.stride(0) % 4 or res.stride(1) % 4:
            res = res.contiguous()
        return res, res.stride(0), res.stride(1), res.shape[1]
    res = res.contiguous().reshape(-1, res.shape[-1])
    return res, 0, res.stride(0), res.shape[0]


def _add_ln_impl(
    x: Tensor,
    bias: Optional[Tensor],
    res: Optional[Tensor],
    gamma: Tensor,
    beta: Tensor,
    eps: float,
    out_dtype: torch.dtype,
) -> tuple[Tensor, Tensor, Tensor]:
    """``y = LayerNorm(x + bias + res) * gamma + beta`` over the last dim;
    returns (y in ``out_dtype``, mean, rstd).  ``res`` has x's shape (a
    broadcast view is read in place)."""
    _eager.refuse_capture("deberta_amd::add_ln")
    C = x.shape[-1]
    xr = _rows(x)
    N = xr.shape[0]
    a = _lib.DsaLnArgs()
    a.x, a.x_stride, a.x_dtype = xr.data_ptr(), xr.stride(0), _dt(x, "add_ln x")
    bias, gamma, beta = _vec(bias), gamma.contiguous(), beta.contiguous()
    a.param_dtype = _dt(gamma, "add_ln gamma")
    for t, n in ((bias, "bias"), (beta, "beta")):
        if t is not None and t.dtype != gamma.dtype:
            raise TypeError(f"add_ln: {n} dtype {t.dtype} differs from gamma's {gamma.dtype}")
    a.bias, a.gamma, a.beta = _ptr(bias), gamma.data_ptr(), beta.data_ptr()
    keep = None
    if res is not None:
        keep, s0, s1, rpg = _res_layout(res, x)
        a.res, a.res_dtype = keep.data_ptr(), _dt(keep, "add_ln res")
        a.res_strides[:] = (s0, s1)
        a.rows_per_group = rpg
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    mean = torch.empty((N,), dtype=torch.float32, device=x.device)
    rstd = torch.empty((N,), dtype=torch.float32, device=x.device)
    a.y, a.y_stride, a.y_dtype = y.data_ptr(), C, _dt(y, "add_ln y")
    a.mean, a.rstd = mean.data_ptr(), rstd.data_ptr()
    a.N, a.C, a.eps = N, C, float(eps)
    _lib.check(_lib.load().dsa_add_ln_fwd(ctypes.byref(a), _stream(x)), "dsa_add_ln_fwd")
    return y, mean, rstd


add_ln = torch.library.custom_op("deberta_amd::add_ln", _add_ln_impl, mutates_args=(), device_types="cuda", tags=_TAGS)


@add_ln.register_fake
def _add_ln_fake(x, bias, res, gamma, beta, eps, out_dtype):
    N = x.numel() // x.shape[-1]
    return x.new_empty(x.shape, dtype=out_dtype), x.new_empty((N,), dtype=torch.float32), x.new_empty((N,), dtype=torch.float32)


def _add_ln_bwd_impl(
    dy: Tensor,
    x: Tensor,
    bias: Optional[Tensor],
    res: Optional[Tensor],
    gamma: Tensor,
    mean: Tensor,
    rstd: Tensor,
    dz_dtype: torch.dtype,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(dz, dgamma, dbeta, dbias): dz the gradient of ``x + bias + res`` in
    ``dz_dtype``; the parameter gradients in gamma's dtype (dbias empty
    without a bias)."""
    _eager.refuse_capture("deberta_amd::add_ln_bwd")
    C = x.shape[-1]
    xr = _rows(x)
    N = xr.shape[0]
    dyr = _rows(dy)
    a = _lib.DsaLnArgs()
    a.x, a.x_stride, a.x_dtype = xr.data_ptr(), xr.stride(0), _dt(x, "add_ln x")
    bias, gamma = _vec(bias), gamma.contiguous()
    a.param_dtype = _dt(gamma, "add_ln gamma")
    a.bias, a.gamma, a.beta = _ptr(bias), gamma.data_ptr(), gamma.data_ptr()
    if res is not None:
        keep, s0, s1, rpg = _res_layout(res, x)
        a.res, a.res_dtype = keep.data_ptr(), _dt(keep, "add_ln res")
        a.res_strides[:] = (s0, s1)
        a.rows_per_group = rpg
    dz = torch.empty(x.shape, dtype=dz_dtype, device=x.device)
    dgamma, dbeta = torch.empty_like(gamma), torch.empty_like(gamma)
    dbias = torch.empty_like(gamma) if bias is not None else gamma.new_empty((0,))
    a.mean, a.rstd = mean.data_ptr(), rstd.data_ptr()
    a.dy, a.dy_stride, a.dy_dtype = dyr.data_ptr(), dyr.stride(0), _dt(dy, "add_ln dy")
    a.dz, a.dz_stride, a.dz_dtype = dz.data_ptr(), C, _dt(dz, "add_ln dz")
    a.dgamma, a.dbeta, a.dbias = dgamma.data_ptr(), dbeta.data_ptr(), _ptr(dbias) if bias is not None else None
    lib = _lib.load()
    nws = lib.dsa_block_workspace_bytes(_lib.DSA_BLOCK_LN, N, C)
    ws = torch.empty((nws,), dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nws
    a.N, a.C = N, C
    _lib.check(lib.dsa_add_ln_bwd(ctypes.byref(a), _stream(x)), "dsa_add_ln_bwd")
    return dz, dgamma, dbeta, dbias


add_ln_bwd = torch.library.custom_op("deberta_amd::add_ln_bwd", _add_ln_bwd_impl, mutates_args=(), device_types="cuda", tags=_TAGS)


@add_ln_bwd.register_fake
def _add_ln_bwd_fake(dy, x, bias, res, gamma, mean, rstd, dz_dtype):
    return (
        x.new_empty(x.shape, dtype=dz_dtype),
        gamma.new_empty(gamma.shape),
        gamma.new_empty(gamma.shape),
        gamma.new_empty(gamma.shape) if bias is not None else gamma.new_empty((0,)),
    )


def _add_ln_setup(ctx, inputs, output):
    x, bias, res, gamma, beta, eps, out_dtype = inputs
    _, mean, rstd = output
    ctx.mark_non_differentiable(mean, rstd)
    ctx.save_for_backward(x, bias, res, gamma, mean, rstd)
    ctx.has_res = res is not None


def _add_ln_backward(ctx, dy, dmean, drstd):
    x, bias, res, gamma, mean, rstd = ctx.saved_tensors
    dz, dgamma, dbeta, dbias = _eager.on_eager(ctx, add_ln_bwd, _add_ln_bwd_impl)(dy, x, bias, res, gamma, mean, rstd, x.dtype)
    dres = None
    if ctx.has_res:
        dres = dz if res.dtype == dz.dtype else dz.to(res.dtype)
    return dz, (dbias if bias is not None else None), dres, dgamma, dbeta, None, None


torch.library.register_autograd("deberta_amd::add_ln", _add_ln_backward, setup_context=_add_ln_setup)
_AddLnFunction = _eager.function("_AddLnFunction", _add_ln_impl, _add_ln_setup, _add_ln_backward)


def call_add_ln(x, bias, res, gamma, beta, eps: float, out_dtype: torch.dtype):
    """``deberta_amd::add_ln`` with its autograd (the implementation in a
    torch.autograd.Function in plain eager mode, the op otherwise)."""
    if _eager.eager(x):
        return _AddLnFunction.apply(x, bias, res, gamma, beta, eps, out_dtype)
    return torch.ops.deberta_amd.add_ln(x, bias, res, gamma, beta, eps, out_dtype)


def _ln_out_dtype(x: Tensor, res: Optional[Tensor]) -> torch.dtype:
    """torch's result dtype for LayerNorm(x + res): float32 under CUDA
    autocast (layer_norm runs in float32 there), else the promoted dtype."""
    if torch.is_autocast_enabled("cuda"):
        return torch.float32
    return x.dtype if res is None else torch.promote_types(x.dtype, res.dtype)


def fused_add_layer_norm(
    x: Tensor, bias: Optional[Tensor], res: Optional[Tensor], ln: nn.LayerNorm
) -> Tensor:
    """``ln(x + bias + res)`` in one kernel (``ln`` an ``nn.LayerNorm`` over
    the last dim, with affine parameters)."""
    if ln.weight is None or ln.bias is None:
        raise ValueError("fused_add_layer_norm needs an affine LayerNorm")
    y, _, _ = call_add_ln(x, bias, res, ln.weight, ln.bias, float(ln.eps), _ln_out_dtype(x, res))
    return y


# ---------------------------------------------------------------------------
# bias + GELU


def _bias_gelu_impl(x: Tensor, bias: Optional[Tensor]) -> Tensor:
    """``gelu(x + bias)`` (erf form) in x's dtype."""
    _eager.refuse_capture("deberta_amd::bias_gelu")
    C = x.shape[-1]
    xr = _rows(x)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    bias = _vec(bias)
    a = _lib.DsaGeluArgs()
    a.x, a.x_stride, a.x_dtype = xr.data_ptr(), xr.stride(0), _dt(x, "bias_gelu x")
    a.bias = _ptr(bias)
    a.param_dtype = _dt(bias, "bias_gelu bias") if bias is not None else _lib.DSA_F32
    a.y, a.y_stride, a.y_dtype = y.data_ptr(), C, a.x_dtype
    a.N, a.C = xr.shape[0], C
    _lib.check(_lib.load().dsa_bias_gelu_fwd(ctypes.byref(a), _stream(x)), "dsa_bias_gelu_fwd")
    return y


bias_gelu = torch.library.custom_op("deberta_amd::bias_gelu", _bias_gelu_impl, mutates_args=(), device_types="cuda", tags=_TAGS)


@bias_gelu.register_fake
def _bias_gelu_fake(x, bias):
    return x.new_empty(x.shape)


def _bias_gelu_bwd_impl(dy: Tensor, x: Tensor, bias: Optional[Tensor]) -> tuple[Tensor, Tensor]:
    """(dz, dbias): the gradient of ``x + bias`` in x's dtype and dbias in
    the bias dtype (empty without a bias)."""
    _eager.refuse_capture("deberta_amd::bias_gelu_bwd")
    C = x.shape[-1]
    xr, dyr = _rows(x), _rows(dy)
    N = xr.shape[0]
    bias = _vec(bias)
    dz = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dbias = torch.empty_like(bias) if bias is not None else x.new_empty((0,))
    a = _lib.DsaGeluArgs()
    a.x, a.x_stride, a.x_dtype = xr.data_ptr(), xr.stride(0), _dt(x, "bias_gelu x")
    a.bias = _ptr(bias)
    a.param_dtype = _dt(bias, "bias_gelu bias") if bias is not None else _lib.DSA_F32
    a.dy, a.dy_stride, a.dy_dtype = dyr.data_ptr(), dyr.stride(0), _dt(dy, "bias_gelu dy")
    a.dz, a.dz_stride, a.dz_dtype = dz.data_ptr(), C, a.x_dtype
    a.dbias = _ptr(dbias) if bias is not None else None
    lib = _lib.load()
    nws = lib.dsa_block_workspace_bytes(_lib.DSA_BLOCK_GELU, N, C)
    ws = torch.empty((nws,), dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nws
    a.N, a.C = N, C
    _lib.check(lib.dsa_bias_gelu_bwd(ctypes.byref(a), _stream(x)), "dsa_bias_gelu_bwd")
    return dz, dbias


bias_gelu_bwd = torch.library.custom_op("deberta_amd::bias_gelu_bwd", _bias_gelu_bwd_impl, mutates_args=(), device_types="cuda", tags=_TAGS)


@bias_gelu_bwd.register_fake
def _bias_gelu_bwd_fake(dy, x, bias):
    return x.new_empty(x.shape), (bias.new_empty(bias.shape) if bias is not None else x.new_empty((0,)))


def _bias_gelu_setup(ctx, inputs, output):
    x, bias = inputs
    ctx.save_for_backward(x, bias)


def _bias_gelu_backward(ctx, dy):
    x, bias = ctx.saved_tensors
    dz, dbias = _eager.on_eager(ctx, bias_gelu_bwd, _bias_gelu_bwd_impl)(dy, x, bias)
    return dz, (dbias if bias is not None else None)


torch.library.register_autograd("deberta_amd::bias_gelu", _bias_gelu_backward, setup_context=_bias_gelu_setup)
_BiasGeluFunction = _eager.function("_BiasGeluFunction", _bias_gelu_impl, _bias_gelu_setup, _bias_gelu_backward)


def call_bias_gelu(x: Tensor, bias: Optional[Tensor]) -> Tensor:
    """``deberta_amd::bias_gelu`` with its autograd (eager: the
    implementation in a torch.autograd.Function)."""
    if _eager.eager(x):
        return _BiasGeluFunction.apply(x, bias)
    return torch.ops.deberta_amd.bias_gelu(x, bias)


# ---------------------------------------------------------------------------
# RTD classifier + BCE


def _rtd_loss_impl(
    x: Tensor, w: Tensor, b: Optional[Tensor], labels: Tensor, active: Optional[Tensor]
) -> tuple[Tensor, Tensor, Tensor]:
    """(loss, logits, denom): ``logits = x @ w + b`` per row (float32) and
    ``loss = sum(active * BCE(logits, labels)) / max(sum(active), 1)``."""
    _eager.refuse_capture("deberta_amd::rtd_loss")
    C = x.shape[-1]
    xr = _rows(x)
    N = xr.shape[0]
    w = w.reshape(-1).contiguous()
    b = None if b is None else b.reshape(-1).contiguous()
    lab = labels.reshape(-1).to(torch.float32).contiguous()
    act = None if active is None else active.reshape(-1).to(torch.uint8).contiguous()
    logits = torch.empty((N,), dtype=torch.float32, device=x.device)
    loss = torch.empty((), dtype=torch.float32, device=x.device)
    denom = torch.empty((), dtype=torch.float32, device=x.device)
    a = _lib.DsaRtdArgs()
    a.x, a.x_stride, a.x_dtype = xr.data_ptr(), xr.stride(0), _dt(x, "rtd_loss x")
    a.w, a.b, a.param_dtype = w.data_ptr(), _ptr(b), _dt(w, "rtd_loss w")
    a.labels, a.active = lab.data_ptr(), _ptr(act)
    a.logits, a.loss, a.denom = logits.data_ptr(), loss.data_ptr(), denom.data_ptr()
    lib = _lib.load()
    nws = lib.dsa_block_workspace_bytes(_lib.DSA_BLOCK_RTD, N, C)
    ws = torch.empty((nws,), dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nws
    a.N, a.C = N, C
    _lib.check(lib.dsa_rtd_loss_fwd(ctypes.byref(a), _stream(x)), "dsa_rtd_loss_fwd")
    return loss, logits.view(x.shape[:-1]), denom


rtd_loss = torch.library.custom_op("deberta_amd::rtd_loss", _rtd_loss_impl, mutates_args=(), device_types="cuda", tags=_TAGS)


@rtd_loss.register_fake
def _rtd_loss_fake(x, w, b, labels, active):
    return (
        x.new_empty((), dtype=torch.float32),
        x.new_empty(x.shape[:-1], dtype=torch.float32),
        x.new_empty((), dtype=torch.float32),
    )


def _rtd_loss_bwd_impl(
    dloss: Tensor, x: Tensor, w: Tensor, b: Optional[Tensor], labels: Tensor, active: Optional[Tensor],
    logits: Tensor, denom: Tensor,
) -> tuple[Tensor, Tensor, Tensor]:
    """(dx, dw, db) of the loss: dx in x's dtype, dw / db in w's dtype (db
    empty without a bias)."""
    _eager.refuse_capture("deberta_amd::rtd_loss_bwd")
    C = x.shape[-1]
    xr = _rows(x)
    N = xr.shape[0]
    wf = w.reshape(-1).contiguous()
    lab = labels.reshape(-1).to(torch.float32).contiguous()
    act = None if active is None else active.reshape(-1).to(torch.uint8).contiguous()
    dl = dloss.reshape(1).to(torch.float32).contiguous()
    lg = logits.reshape(-1).contiguous()
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dw = torch.empty_like(w)
    db = torch.empty_like(b) if b is not None else w.new_empty((0,))
    a = _lib.DsaRtdArgs()
    a.x, a.x_stride, a.x_dtype = xr.data_ptr(), xr.stride(0), _dt(x, "rtd_loss x")
    a.w, a.b, a.param_dtype = wf.data_ptr(), _ptr(b), _dt(w, "rtd_loss w")
    a.labels, a.active = lab.data_ptr(), _ptr(act)
    a.logits, a.denom, a.dloss = lg.data_ptr(), denom.data_ptr(), dl.data_ptr()
    a.dx, a.dx_stride, a.dx_dtype = dx.data_ptr(), C, a.x_dtype
    a.dw, a.db = dw.data_ptr(), _ptr(db) if b is not None else None
    lib = _lib.load()
    nws = lib.dsa_block_workspace_bytes(_lib.DSA_BLOCK_RTD, N, C)
    ws = torch.empty((nws,), dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nws
    a.N, a.C = N, C
    _lib.check(lib.dsa_rtd_loss_bwd(ctypes.byref(a), _stream(x)), "dsa_rtd_loss_bwd")
    return dx, dw, db


rtd_loss_bwd = torch.library.custom_op("deberta_amd::rtd_loss_bwd", _rtd_loss_bwd_impl, mutates_args=(), device_types="cuda", tags=_TAGS)


@rtd_loss_bwd.register_fake
def _rtd_loss_bwd_fake(dloss, x, w, b, labels, active, logits, denom):
    return x.new_empty(x.shape), w.new_empty(w.shape), (b.new_empty(b.shape) if b is not None else w.new_empty((0,)))


def _rtd_setup(ctx, inputs, output):
    x, w, b, labels, active = inputs
    _, logits, denom = output
    ctx.mark_non_differentiable(logits, denom)
    ctx.save_for_backward(x, w, b, labels, active, logits, denom)
    ctx.set_materialize_grads(False)


def _rtd_backward(ctx, dloss, dlogits, ddenom):
    x, w, b, labels, active, logits, denom = ctx.saved_tensors
    if dloss is None:
        return None, None, None, None, None
    dx, dw, db = _eager.on_eager(ctx, rtd_loss_bwd, _rtd_loss_bwd_impl)(dloss, x, w, b, labels, active, logits, denom)
    return dx, dw, (db if b is not None else None), None, None


torch.library.register_autograd("deberta_amd::rtd_loss", _rtd_backward, setup_context=_rtd_setup)
_RtdLossFunction = _eager.function("_RtdLossFunction", _rtd_loss_impl, _rtd_setup, _rtd_backward)


def call_rtd_loss(x: Tensor, w: Tensor, b: Optional[Tensor], labels: Tensor, active: Optional[Tensor]):
    """``deberta_amd::rtd_loss`` with its autograd (eager: the
    implementation in a torch.autograd.Function)."""
    if _eager.eager(x):
        return _RtdLossFunction.apply(x, w, b, labels, active)
    return torch.ops.deberta_amd.rtd_loss(x, w, b, labels, active)


# ---------------------------------------------------------------------------
# modules


def _on_gpu(t: Tensor) -> bool:
    return t.device.type == "cuda"


def _bce_loss(logits: Tensor, labels: Tensor, active: Optional[Tensor]) -> Tensor:
    """The discriminator loss in torch operations (rtd.py:1129-1139): BCE with
    logits per token in float32, summed over the active tokens, over
    max(#active, 1)."""
    act = torch.ones_like(logits, dtype=torch.float32) if active is None else active.to(torch.float32)
    per_token = F.binary_cross_entropy_with_logits(logits.float(), labels.float(), reduction="none")
    return (per_token * act).sum() / act.sum().clamp(min=1.0)


class FusedSelfOutput(nn.Module):
    """DebertaV2SelfOutput (deberta_v2_native.py:115-165): ``LayerNorm(
    dense(hidden) + input)``, the dense GEMM without its bias and the bias,
    residual and LayerNorm in one kernel."""

    def __init__(self, config: Any, in_features: Optional[int] = None) -> None:
        super().__init__()
        hidden = int(config.hidden_size)
        self.dense = nn.Linear(int(in_features or hidden), hidden)
        self.LayerNorm = nn.LayerNorm(hidden, eps=float(getattr(config, "layer_norm_eps", 1e-7)))
        self.dropout = nn.Dropout(float(getattr(config, "hidden_dropout_prob", 0.0)))

    def forward(self, hidden_states: Tensor, input_tensor: Tensor) -> Tensor:
        if not _on_gpu(hidden_states):  # the reference's block in torch operations
            return self.LayerNorm(self.dropout(self.dense(hidden_states)) + input_tensor)
        if self.training and self.dropout.p > 0.0:
            # dropout acts on dense(x) with its bias: torch's dropout, then
            # the residual LayerNorm in one kernel
            return fused_add_layer_norm(self.dropout(self.dense(hidden_states)), None, input_tensor, self.LayerNorm)
        # the bias is added in float32 inside the LayerNorm kernel (in its
        # own dtype, the LayerNorm's)
        x = F.linear(hidden_states, self.dense.weight)
        return fused_add_layer_norm(x, self.dense.bias, input_tensor, self.LayerNorm)


class FusedOutput(FusedSelfOutput):
    """DebertaV2Output (deberta_v2_native.py:733-758): the FFN's output
    projection, then bias + residual + LayerNorm in one kernel."""

    def __init__(self, config: Any) -> None:
        super().__init__(config, in_features=int(config.intermediate_size))


class FusedIntermediate(nn.Module):
    """DebertaV2Intermediate (deberta_v2_native.py:703-730) with
    ``hidden_act = "gelu"``: the dense GEMM without its bias, then bias +
    GELU in one kernel."""

    def __init__(self, config: Any) -> None:
        super().__init__()
        act = getattr(config, "hidden_act", "gelu")
        if act != "gelu":
            raise NotImplementedError(f"FusedIntermediate supports hidden_act 'gelu', got {act!r}")
        self.dense = nn.Linear(int(config.hidden_size), int(config.intermediate_size))

    def forward(self, hidden_states: Tensor) -> Tensor:
        if not _on_gpu(hidden_states):
            return F.gelu(self.dense(hidden_states))
        x = F.linear(hidden_states, self.dense.weight)
        bias = self.dense.bias
        if bias is not None:
            bias = bias.to(x.dtype)
        return call_bias_gelu(x, bias)


class FusedRTDHead(nn.Module):
    """RTDHead (rtd.py:550-626): ``classifier(gelu(dense(LayerNorm(hidden +
    hidden[:, 0]))))``, with the LayerNorm of the CLS-conditioned states in
    one kernel (the CLS row read in place) and dense + bias + GELU in
    another; ``forward_loss`` also fuses the classifier with the
    discriminator's BCE loss (rtd.py:1134-1139)."""

    def __init__(self, config: Any) -> None:
        super().__init__()
        hidden = int(config.hidden_size)
        act = getattr(config, "hidden_act", "gelu")
        if act != "gelu":
            raise NotImplementedError(f"FusedRTDHead supports hidden_act 'gelu', got {act!r}")
        if bool(getattr(config, "use_rmsnorm_heads", False)):
            raise NotImplementedError("FusedRTDHead supports the LayerNorm head (use_rmsnorm_heads=False)")
        self.dense = nn.Linear(hidden, hidden)
        self.act = nn.GELU()
        eps = float(getattr(config, "norm_eps", getattr(config, "layer_norm_eps", 1e-6)))
        self.norm = nn.LayerNorm(hidden, eps=eps)
        self.classifier = nn.Linear(hidden, 1)

    @staticmethod
    def _use_global_cls_context(attention_mask: Optional[Tensor]) -> bool:
        """The reference's rule (rtd.py:584-603): no CLS context under
        pairwise masks with an explicit query axis."""
        if attention_mask is None:
            return True
        mask = attention_mask
        if mask.ndim == 4:
            mask = mask[:, 0] if mask.shape[1] == 1 else mask.any(dim=1)
        return not (mask.ndim == 3 and mask.shape[-2] != 1)

    def _features(self, hidden_states: Tensor, attention_mask: Optional[Tensor]) -> Tensor:
        res = None
        if self._use_global_cls_context(attention_mask):
            res = hidden_states[:, 0:1, :].expand(hidden_states.shape)
        if not _on_gpu(hidden_states):  # the reference's head in torch operations
            x = self.norm(hidden_states + res if res is not None else hidden_states)
            return self.act(self.dense(x))
        x = fused_add_layer_norm(hidden_states, None, res, self.norm)
        x = F.linear(x, self.dense.weight)
        bias = self.dense.bias
        if bias is not None:
            bias = bias.to(x.dtype)
        return call_bias_gelu(x, bias)

    def forward(self, hidden_states: Tensor, attention_mask: Optional[Tensor] = None) -> Tensor:
        """Per-token logits ``(B, S)``."""
        return F.linear(self._features(hidden_states, attention_mask), self.classifier.weight, self.classifier.bias).squeeze(-1)

    def forward_loss(
        self,
        hidden_states: Tensor,
        labels: Tensor,
        active: Optional[Tensor] = None,
        attention_mask: Optional[Tensor] = None,
    ) -> tuple[Tensor, Tensor]:
        """(loss, logits): the discriminator loss ``sum(active * BCE(logits,
        labels)) / max(sum(active), 1)`` and the float32 logits, the
        classifier and the loss in one kernel."""
        x = self._features(hidden_states, attention_mask)
        if not _on_gpu(x):
            logits = self.classifier(x).squeeze(-1).float()
            return _bce_loss(logits, labels, active), logits
        w = self.classifier.weight.reshape(-1)
        b = self.classifier.bias
        if b is not None:
            b = b.to(w.dtype)
        loss, logits, _ = call_rtd_loss(x, w, b, labels, active)
        return loss, logits


class RelativeEmbeddings(nn.Module):
    """The encoder's shared relative-embedding table and its LayerNorm
    (deberta_v2_native.py:1036-1047, ``norm_rel_ebd`` with ``layer_norm``):
    ``forward()`` returns ``LayerNorm(rel_embeddings.weight)`` from one
    kernel.  The attention layers then project it for c2p / p2c / p2p with
    one GEMM per layer (``DisentangledSelfAttention._relative_tables``)."""

    def __init__(self, config: Any) -> None:
        super().__init__()
        hidden = int(config.hidden_size)
        buckets = int(getattr(config, "position_buckets", -1))
        max_rel = int(getattr(config, "max_relative_positions", -1))
        if max_rel < 1:
            max_rel = int(config.max_position_embeddings)
        pos_ebd = buckets if buckets > 0 else max_rel
        self.rel_embeddings = nn.Embedding(pos_ebd * 2, hidden)
        self.LayerNorm = nn.LayerNorm(hidden, eps=float(getattr(config, "layer_norm_eps", 1e-7)), elementwise_affine=True)

    def forward(self) -> Tensor:
        w = self.rel_embeddings.weight
        if not _on_gpu(w):
            return self.LayerNorm(w)
        return fused_add_layer_norm(w, None, None, self.LayerNorm)
