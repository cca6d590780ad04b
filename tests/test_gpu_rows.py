"""The row kernels of include/dsa_block.h (add + LayerNorm, bias + GELU, the
RTD classifier + BCE loss) at every row width class and every element-type
combination the C-ABI accepts, called through the C-ABI.

The kernels are templates over the 4-element chunks a lane holds (NC =
ceil(C / 256): 1, 2, 3, 4, 6, 8 for C up to 2048) and over the dtypes of
x, the residual, y, dy and dx, each float32 or bfloat16.  Rows are 70 (not
a multiple of any kernel's rows per block); C = 300 and 1300 leave partial
chunks.  References are float64 on the CPU from the values the kernels
read: torch's layer_norm and autograd (deberta_v2_native.py:115-165 add the
residual before the LayerNorm), the erf GELU and its derivative
(:703-730), and the masked BCE-with-logits mean (rtd.py:1134-1139).  Bounds:
outputs in float32 to 1e-5 of scale, in bfloat16 to 2^-7 of scale (one
rounding of a float32 result is at most 2^-9).
"""

from __future__ import annotations

import ctypes
import itertools
import math

import pytest
import torch

from deberta_amd import _lib

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16
_CODE = {F32: _lib.DSA_F32, BF16: _lib.DSA_BF16}
_WIDTHS = [128, 300, 512, 768, 1024, 1300, 2048]  # NC = 1, 2, 2, 3, 4, 6, 8
_N = 70


def _bound(dtype: torch.dtype) -> float:
    return 1e-5 if dtype == F32 else 2.0**-7


def _err(got: torch.Tensor, want: torch.Tensor) -> float:
    scale = float(want.abs().max())
    return float((got.double().cpu() - want).abs().max()) / max(scale, 1e-30)


def _mk(shape, dtype, gen, dev, scale=1.0, shift=0.0):
    t = torch.randn(*shape, generator=gen, dtype=torch.float64) * scale + shift
    t = t.to(dtype)
    return t.to(dev), t.double()


def _call(fn, a, dev):
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(getattr(lib, fn)(ctypes.byref(a), stream), fn)
    torch.cuda.synchronize(dev)


def _workspace(kind, N, C, dev):
    n = _lib.load().dsa_block_workspace_bytes(kind, N, C)
    return torch.empty((max(n, 1),), dtype=torch.uint8, device=dev)


_LN_COMBOS = list(itertools.product([F32, BF16], repeat=3))


@pytest.mark.parametrize("C", _WIDTHS)
@pytest.mark.parametrize("xd,rd,yd", _LN_COMBOS, ids=lambda d: "bf16" if d == BF16 else "fp32")
def test_add_ln_widths_and_dtypes(C, xd, rd, yd, gpu):
    """y = LayerNorm(x + bias + res) * gamma + beta and its backward (dz in
    x's dtype from dy in y's dtype; dgamma, dbeta, dbias in the parameters'
    dtype), for x, res and y each float32 or bfloat16."""
    pd = F32 if (C // 4) % 2 else BF16
    g = torch.Generator().manual_seed(C * 8 + _LN_COMBOS.index((xd, rd, yd)))
    x, x64 = _mk((_N, C), xd, g, gpu, 1.0, 0.3)
    res, res64 = _mk((_N, C), rd, g, gpu, 0.5)
    bias, bias64 = _mk((C,), pd, g, gpu, 0.1)
    gamma, gamma64 = _mk((C,), pd, g, gpu, 0.2, 1.0)
    beta, beta64 = _mk((C,), pd, g, gpu, 0.1)
    dy, dy64 = _mk((_N, C), yd, g, gpu)
    eps = 1e-7
    y = torch.empty((_N, C), dtype=yd, device=gpu)
    mean = torch.empty((_N,), dtype=F32, device=gpu)
    rstd = torch.empty((_N,), dtype=F32, device=gpu)
    a = _lib.DsaLnArgs()
    a.x, a.x_stride, a.x_dtype = x.data_ptr(), C, _CODE[xd]
    a.bias, a.gamma, a.beta, a.param_dtype = bias.data_ptr(), gamma.data_ptr(), beta.data_ptr(), _CODE[pd]
    a.res, a.res_dtype, a.rows_per_group = res.data_ptr(), _CODE[rd], _N
    a.res_strides[:] = (0, C)
    a.y, a.y_stride, a.y_dtype = y.data_ptr(), C, _CODE[yd]
    a.mean, a.rstd = mean.data_ptr(), rstd.data_ptr()
    a.N, a.C, a.eps = _N, C, eps
    _call("dsa_add_ln_fwd", a, gpu)

    dz = torch.empty((_N, C), dtype=xd, device=gpu)
    grads = [torch.empty((C,), dtype=pd, device=gpu) for _ in range(3)]
    ws = _workspace(_lib.DSA_BLOCK_LN, _N, C, gpu)
    a.dy, a.dy_stride, a.dy_dtype = dy.data_ptr(), C, _CODE[yd]
    a.dz, a.dz_stride, a.dz_dtype = dz.data_ptr(), C, _CODE[xd]
    a.dgamma, a.dbeta, a.dbias = (t.data_ptr() for t in grads)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _call("dsa_add_ln_bwd", a, gpu)

    z = (x64 + bias64 + res64).requires_grad_(True)
    gam, bet = gamma64.clone().requires_grad_(True), beta64.clone().requires_grad_(True)
    want = torch.nn.functional.layer_norm(z, (C,), gam, bet, eps)
    dz64, dg64, db64 = torch.autograd.grad(want, [z, gam, bet], dy64)
    errs = {
        "y": _err(y, want.detach()),
        "mean": _err(mean, z.detach().mean(-1)),
        "rstd": _err(rstd, 1 / torch.sqrt(z.detach().var(-1, unbiased=False) + eps)),
        "dz": _err(dz, dz64),
        "dgamma": _err(grads[0], dg64),
        "dbeta": _err(grads[1], db64),
        "dbias": _err(grads[2], dz64.sum(0)),
    }
    bounds = {"y": _bound(yd), "mean": 1e-5, "rstd": 1e-5, "dz": _bound(xd)}
    bounds.update({k: _bound(pd) for k in ("dgamma", "dbeta", "dbias")})
    bad = {k: (e, bounds[k]) for k, e in errs.items() if not e <= bounds[k]}
    assert not bad, (C, xd, rd, yd, pd, bad)


def _gelu64(z):
    return 0.5 * z * (1 + torch.erf(z / math.sqrt(2)))


def _dgelu64(z):
    return 0.5 * (1 + torch.erf(z / math.sqrt(2))) + z * torch.exp(-0.5 * z * z) / math.sqrt(2 * math.pi)


@pytest.mark.parametrize("C", [300, 1024, 1304])  # 300: the 4-wide kernels; 1024, 1304: the 8-wide
@pytest.mark.parametrize("xd,yd", list(itertools.product([F32, BF16], repeat=2)), ids=lambda d: "bf16" if d == BF16 else "fp32")
def test_bias_gelu_dtypes(C, xd, yd, gpu):
    """y = gelu(x + bias) in y's dtype, and dz = dy * gelu'(x + bias) in
    x's dtype from dy in y's dtype, dbias the column sums of dz."""
    pd = BF16 if xd == yd else F32
    g = torch.Generator().manual_seed(C + 7 * (xd == BF16) + 3 * (yd == BF16))
    x, x64 = _mk((_N, C), xd, g, gpu, 2.0)
    bias, bias64 = _mk((C,), pd, g, gpu, 0.3)
    dy, dy64 = _mk((_N, C), yd, g, gpu)
    y = torch.empty((_N, C), dtype=yd, device=gpu)
    a = _lib.DsaGeluArgs()
    a.x, a.x_stride, a.x_dtype = x.data_ptr(), C, _CODE[xd]
    a.bias, a.param_dtype = bias.data_ptr(), _CODE[pd]
    a.y, a.y_stride, a.y_dtype = y.data_ptr(), C, _CODE[yd]
    a.N, a.C = _N, C
    _call("dsa_bias_gelu_fwd", a, gpu)
    dz = torch.empty((_N, C), dtype=xd, device=gpu)
    dbias = torch.empty((C,), dtype=pd, device=gpu)
    ws = _workspace(_lib.DSA_BLOCK_GELU, _N, C, gpu)
    a.dy, a.dy_stride, a.dy_dtype = dy.data_ptr(), C, _CODE[yd]
    a.dz, a.dz_stride, a.dz_dtype = dz.data_ptr(), C, _CODE[xd]
    a.dbias = dbias.data_ptr()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _call("dsa_bias_gelu_bwd", a, gpu)
    z = x64 + bias64
    dz64 = dy64 * _dgelu64(z)
    errs = {"y": _err(y, _gelu64(z)), "dz": _err(dz, dz64), "dbias": _err(dbias, dz64.sum(0))}
    bounds = {"y": _bound(yd), "dz": _bound(xd), "dbias": _bound(pd)}
    bad = {k: (e, bounds[k]) for k, e in errs.items() if not e <= bounds[k]}
    assert not bad, (C, xd, yd, pd, bad)


@pytest.mark.parametrize("C", _WIDTHS)
@pytest.mark.parametrize("xd,dxd", list(itertools.product([F32, BF16], repeat=2)), ids=lambda d: "bf16" if d == BF16 else "fp32")
def test_rtd_loss_widths_and_dtypes(C, xd, dxd, gpu):
    """logits = x . w + b per row and loss = sum(active * BCE) / max(sum
    active, 1); the backward's dx (in dx's dtype), dw and db."""
    pd = F32 if xd == dxd else BF16
    g = torch.Generator().manual_seed(3 * C + 2 * (xd == BF16) + (dxd == BF16))
    x, x64 = _mk((_N, C), xd, g, gpu)
    w, w64 = _mk((C,), pd, g, gpu, 1 / math.sqrt(C))
    b, b64 = _mk((1,), pd, g, gpu, 0.5)
    labels = (torch.rand(_N, generator=g) < 0.3).float()
    active = torch.rand(_N, generator=g) < 0.8
    lab_d, act_d = labels.to(gpu), active.to(torch.uint8).to(gpu)
    logits = torch.empty((_N,), dtype=F32, device=gpu)
    loss = torch.empty((1,), dtype=F32, device=gpu)
    denom = torch.empty((1,), dtype=F32, device=gpu)
    ws = _workspace(_lib.DSA_BLOCK_RTD, _N, C, gpu)
    a = _lib.DsaRtdArgs()
    a.x, a.x_stride, a.x_dtype = x.data_ptr(), C, _CODE[xd]
    a.w, a.b, a.param_dtype = w.data_ptr(), b.data_ptr(), _CODE[pd]
    a.labels, a.active = lab_d.data_ptr(), act_d.data_ptr()
    a.logits, a.loss, a.denom = logits.data_ptr(), loss.data_ptr(), denom.data_ptr()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.N, a.C = _N, C
    _call("dsa_rtd_loss_fwd", a, gpu)
    dloss = torch.tensor([0.75], dtype=F32, device=gpu)
    dx = torch.empty((_N, C), dtype=dxd, device=gpu)
    dw = torch.empty((C,), dtype=pd, device=gpu)
    db = torch.empty((1,), dtype=pd, device=gpu)
    a.dloss = dloss.data_ptr()
    a.dx, a.dx_stride, a.dx_dtype = dx.data_ptr(), C, _CODE[dxd]
    a.dw, a.db = dw.data_ptr(), db.data_ptr()
    _call("dsa_rtd_loss_bwd", a, gpu)

    xr, wr, br = x64.clone().requires_grad_(True), w64.clone().requires_grad_(True), b64.clone().requires_grad_(True)
    lg = xr @ wr + br
    act = active.double()
    n = max(float(act.sum()), 1.0)
    bce = torch.nn.functional.binary_cross_entropy_with_logits(lg, labels.double(), reduction="none")
    want = (bce * act).sum() / n
    dx64, dw64, db64 = torch.autograd.grad(want * 0.75, [xr, wr, br])
    errs = {
        "logits": _err(logits, lg.detach()),
        "loss": _err(loss, want.detach().reshape(1)),
        "denom": _err(denom, torch.tensor([n], dtype=torch.float64)),
        "dx": _err(dx, dx64),
        "dw": _err(dw, dw64),
        "db": _err(db, db64),
    }
    bounds = {"logits": 1e-5, "loss": 1e-5, "denom": 0.0, "dx": _bound(dxd), "dw": _bound(pd), "db": _bound(pd)}
    bad = {k: (e, bounds[k]) for k, e in errs.items() if not e <= bounds[k]}
    assert not bad, (C, xd, dxd, pd, bad)
