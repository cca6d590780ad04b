"""Kernel variants that the rest of the GPU suite does not launch.

The kernels are templates over the element type, the head dim, the mask
form, the p2p query rows (``qc``) and dropout, and a kernel trace of the
other GPU tests showed these instantiations never running:

* the forward with ``qc`` (the p2p term, deberta_v2_native.py:298-347,
  carried by the c2p term's query rows) under a key-padding, dense pair or
  segment mask, with and without dropout, at head dims 32 and 64, fp32 and
  bf16, and the backward's fused dq|table kernel with ``qc`` under the
  listed (key-padding or segment) masks;
* the separate dq kernel with ``qc`` and the separate table kernel, listed
  or not, of the stage-split backward (include/dsa.h: DQ, TABLE).

Op-level cases are held to the sweep's bounds: fp32 to 1e-4 of each
tensor's scale (1e-6 absolute where the oracle's value is zero), bf16 to
2e-2 absolute or, where bf16 arithmetic itself passes that, to 1.5x the
reference's own bf16 error on the same case (the oracle's op chain under
bf16 autocast).  Stage-split runs equal the one-call backward: dq, dk, dv
and the gradient of qc bitwise, the table gradients up to the order of
their fp32 atomic additions (1e-5 of scale).
"""

from __future__ import annotations

import ctypes
import math
import sys

import pytest
import torch

from tests._cases import Case, hip_run, make_inputs, max_abs, max_rel, oracle_run
from tests.test_gpu_precision import _reference_bf16

pytestmark = pytest.mark.gpu

_P2P_TYPES = ["c2p|p2c|p2p", "p2p", "c2p|p2p", "p2c|p2p"]
_BUCKETS = [(256, 512), (32, 64), (-1, 130), (64, 512)]
_LENGTHS = [300, 129, 517, 64, 260, 33, 411, 200]


def _say(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _p2p_cases() -> list[tuple[Case, torch.dtype]]:
    cases, i = [], 0
    for dtype in (torch.float32, torch.bfloat16):
        for D in (32, 64):
            for mask in ("none", "key", "pair", "seg"):
                for dropout in (0.0, 0.1):
                    buckets, max_pos = _BUCKETS[(i // 2) % 4]
                    c = Case(
                        B=2, H=2, L=_LENGTHS[i % 8], D=D, buckets=buckets, max_pos=max_pos,
                        types=_P2P_TYPES[(i + i // 8) % 4], mask=mask, seed=90000 + i, dropout=dropout,
                    )
                    cases.append((c, dtype))
                    i += 1
    return cases


_CASES = _p2p_cases()


def _check(c: Case, x: dict, ref: dict, got: dict, dtype: torch.dtype) -> dict:
    errs, ref16 = {}, None
    for k in ref:
        assert torch.isfinite(got[k]).all(), k
        scale = float(ref[k].abs().max()) if ref[k].numel() else 0.0
        if dtype == torch.float32:
            e = max_rel(got[k], ref[k]) if scale > 1e-6 else max_abs(got[k], ref[k])
            errs[k] = e
            assert e <= 1e-4, (c, k, e)
        else:
            e = errs[k] = max_abs(got[k], ref[k])
            if e > 2e-2:
                if ref16 is None:
                    ref16 = _reference_bf16(c, x)
                theirs = max_abs(ref16[k], ref[k])
                _say(f"[variants] {c} {k}: {e:.4f} against the reference's bf16 {theirs:.4f}")
                assert e <= 1.5 * theirs, (c, k, e, theirs)
    return errs


@pytest.mark.parametrize(
    "c,dtype", _CASES,
    ids=[f"{'bf16' if d == torch.bfloat16 else 'fp32'}-D{c.D}-{c.mask}-{c.types}-p{c.dropout}" for c, d in _CASES],
)
def test_p2p_op_variants(c, dtype, gpu):
    """The op with the p2p term against the oracle, forward and every
    gradient (q, k, v, both tables), under every mask form and dropout."""
    x = make_inputs(c)
    ref = oracle_run(c, x, dtype)
    got = hip_run(c, x, dtype, gpu)
    errs = _check(c, x, ref, got, dtype)
    _say(f"[p2p variants] {c} {errs}")


def _segment_ids(B: int, L: int) -> torch.Tensor:
    """Packed documents of 37, 90, 5, ... tokens and a padded tail (id 0)
    in row 1."""
    ids = torch.zeros(B, L, dtype=torch.int64)
    for b in range(B):
        pos, doc = 0, 1
        for n in [37, 90, 5, 120, 61, 200][b:] * 4:
            if pos >= L:
                break
            ids[b, pos : pos + n] = doc
            pos, doc = pos + n, doc + 1
    ids[1, L - 23 :] = 0
    return ids


_STAGE_VARIANTS = [("key", False, 0.0), ("key", True, 0.1), ("seg", True, 0.0), ("seg", False, 0.1), ("none", True, 0.0)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("mask,p2p,dropout", _STAGE_VARIANTS, ids=[f"{m}-p2p{int(p)}-p{d}" for m, p, d in _STAGE_VARIANTS])
def test_stage_split_variants(mask, p2p, dropout, D, dtype, gpu):
    """dsa_bwd as PREP, DKDV, DQ, TABLE and SUM in five calls (the separate
    dq and table kernels) against the one-call backward (the fused
    dq|table kernel), with masks, the p2p query rows and dropout."""
    from deberta_amd import _lib, ops
    from deberta_amd.attention import relative_operands
    from deberta_amd.masks import SegmentMask, kernel_masks
    from deberta_amd.relpos import relative_offset_table

    lib = _lib.load()
    B, L, H, A = 2, 300, 2, 64
    g = torch.Generator().manual_seed(41 + D)
    mk = lambda *s: torch.randn(*s, generator=g).to(gpu, dtype)
    q, k, v, dout = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, 2 * A, D), mk(H, 2 * A, D)
    table = relative_offset_table(L, L, bucket_size=A, max_position=256, device=gpu)
    if mask == "key":
        keep = torch.ones(B, L, dtype=torch.bool)
        keep[1, 190:] = False
        m = keep[:, None, None, :].to(gpu)
    elif mask == "seg":
        m = SegmentMask(_segment_ids(B, L).to(gpu))
    else:
        m = None
    kk, pk = kernel_masks(m, B, L, L, gpu)
    if mask != "none":
        assert kk is not None and pk is None  # the listed form
    qc = relative_operands(["c2p", "p2c", "p2p"], q, kr, qr, A)[2].contiguous() if p2p else None
    scale = 1 / math.sqrt(D * (4 if p2p else 3))
    drop_t = ops.dropout_threshold(dropout) if dropout else 0
    seed = torch.tensor([0x5EED_0F_5747E5], dtype=torch.int64) if drop_t else None
    out, lse, bias, aux = torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, kk, pk, A, scale, True, qc, drop_t, seed)
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    bits = {"PREP": _lib.DSA_STAGE_PREP, "DQ": _lib.DSA_STAGE_DQ, "DKDV": _lib.DSA_STAGE_DKDV,
            "TABLE": _lib.DSA_STAGE_TABLE, "SUM": _lib.DSA_STAGE_SUM}

    def run(calls):
        grads = [torch.full_like(q, float("nan")) for _ in range(3)]
        dqc = torch.full_like(q, float("nan")) if p2p else None
        tabs = [torch.zeros((H, 2 * A, D), dtype=torch.float32, device=gpu) for _ in range(2)]
        a = ops.fill_bwd_args(dout, q, k, v, kr, qr, table, kk, pk, out, lse, bias, A, scale, *grads, *tabs,
                              qc=qc, dqc=dqc, dropout_t=drop_t, dropout_seed=seed, dropout_bits=aux)
        ws = torch.empty((ops.bwd_workspace_bytes(a),), dtype=torch.uint8, device=gpu)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        for c in calls:
            a.stages = 0
            for s in c.split("|") if c else []:
                a.stages |= bits[s]
            _lib.check(lib.dsa_bwd(ctypes.byref(a), stream), "dsa_bwd")
        torch.cuda.synchronize(gpu)
        return dict(zip(["dq", "dk", "dv", "dkr", "dqr", "dqc"], grads + tabs + [dqc]))

    _say(f"[stage variants] {dtype} D={D} mask={mask} p2p={p2p} dropout={dropout}")
    ref = run([""])
    got = run(["PREP", "DKDV", "DQ", "TABLE", "SUM"])
    for name in ref:
        a, b = got[name], ref[name]
        if b is None:
            continue
        assert torch.isfinite(b).all(), f"{name}: the one-call backward left non-finite values"
        if name in ("dkr", "dqr"):
            err = float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
            assert err <= 1e-5, f"{name} differs from the one-call backward ({err:.3e})"
        else:
            assert torch.equal(a, b), f"{name} differs from the one-call backward"
