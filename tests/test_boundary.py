"""CPU checks of the drop-in boundary: the C ABI of libdsa.so (exports and
struct layout against include/dsa.h), the torch.library ops (registration,
fake-tensor shapes, tracing, loud failure off the GPU) and the host-side
mirror of the reference interface (kernel selector, masks, module layout).
No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

import deberta_amd
from deberta_amd import _lib, ops
from deberta_amd.attention import DisentangledSelfAttention
from deberta_amd.config import normalize_attention_kernel, normalize_pos_att_type
from deberta_amd.masks import SegmentMask, build_doc_block_mask, get_attention_mask, kernel_masks, normalize_keep_mask
from oracle import eager

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dsa.h"


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[a-z_]+)\s*\([^;{]*\)\s*;", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built (run python -m deberta_amd._build)")
    return _lib.load()


def test_header_declares_the_abi():
    assert _declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
        for name in _declared_functions():
            assert re.search(rf"\bT {name}$", out, re.M), name


def test_version_and_error_buffer(lib):
    assert lib.dsa_version() == _lib.EXPECTED_VERSION
    assert _lib.last_error() == ""


def test_argument_errors_return_codes_without_launching(lib):
    """Validation happens before any device work, so it is testable here."""
    assert lib.dsa_fwd(None, None) != 0
    assert "null arguments" in _lib.last_error()
    a = _lib.DsaFwdArgs()
    a.B, a.H, a.Lq, a.Lk, a.D, a.dtype = 1, 1, 8, 8, 48, _lib.DSA_BF16
    assert lib.dsa_fwd(ctypes.byref(a), None) != 0
    assert "head dim must be 32 or 64" in _lib.last_error()
    a.D = 64
    assert lib.dsa_fwd(ctypes.byref(a), None) != 0
    assert "required" in _lib.last_error()
    a.dtype = 7
    assert lib.dsa_fwd(ctypes.byref(a), None) != 0
    assert "unsupported dtype" in _lib.last_error()


def test_backward_stage_bits(lib):
    """The stage constants of include/dsa.h and the package agree, and bits
    outside them are refused before any device work."""
    text = (ROOT / "include" / "dsa.h").read_text()
    found = dict((m.group(1), int(m.group(2))) for m in re.finditer(r"(DSA_STAGE_[A-Z]+) = (\d+)", text))
    assert found == {n: getattr(_lib, n) for n in found}
    assert set(found) == {"DSA_STAGE_PREP", "DSA_STAGE_DQ", "DSA_STAGE_DKDV", "DSA_STAGE_FOLD", "DSA_STAGE_TABLE", "DSA_STAGE_SUM"}
    a = _lib.DsaBwdArgs()
    a.stages = 64
    assert lib.dsa_bwd(ctypes.byref(a), None) != 0
    assert "unknown backward stage bits 0x40" in _lib.last_error()


def test_forward_workspace_bytes(lib):
    """The forward's optional scratch: the launch order under key-padding and
    segment masks (two ints per (batch row, 128-query tile), 256-byte
    aligned), then one k-step copy of each relative table in use
    (H * 2A * D elements, 256-byte aligned); nothing without either."""
    a = _lib.DsaFwdArgs()
    a.B, a.H, a.Lq, a.Lk, a.D, a.dtype, a.att_span = 2, 12, 512, 512, 64, _lib.DSA_BF16, 256
    a.flags = 0
    assert lib.dsa_fwd_workspace_bytes(ctypes.byref(a)) == 0
    table = 12 * 512 * 64 * 2
    a.flags = _lib.DSA_C2P | _lib.DSA_P2C
    assert lib.dsa_fwd_workspace_bytes(ctypes.byref(a)) == 2 * table
    a.flags = _lib.DSA_P2C
    assert lib.dsa_fwd_workspace_bytes(ctypes.byref(a)) == table
    a.dtype = _lib.DSA_F32
    assert lib.dsa_fwd_workspace_bytes(ctypes.byref(a)) == 2 * table
    a.dtype, a.flags = _lib.DSA_BF16, _lib.DSA_C2P | _lib.DSA_P2C
    kk = ctypes.create_string_buffer(2 * 512)
    a.key_keep = ctypes.cast(kk, ctypes.c_void_p).value
    order = (2 * 2 * 4 * 4 + 255) // 256 * 256  # cost and order of 2 x 4 items
    assert lib.dsa_fwd_workspace_bytes(ctypes.byref(a)) == order + 2 * table


C_LAYOUT_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "dsa.h"
#define F(s, f) printf(#s "." #f " %zu\n", offsetof(s, f));
int main(void) {
  printf("dsa_fwd_args %zu\n", sizeof(dsa_fwd_args));
  printf("dsa_bwd_args %zu\n", sizeof(dsa_bwd_args));
  %FIELDS%
  return 0;
}
"""


def test_ctypes_structs_match_the_c_header(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    lines = []
    for cname, st in (("dsa_fwd_args", _lib.DsaFwdArgs), ("dsa_bwd_args", _lib.DsaBwdArgs)):
        for fname, _ in st._fields_:
            lines.append(f"F({cname}, {fname})")
    src = tmp_path / "probe.c"
    src.write_text(C_LAYOUT_PROBE.replace("%FIELDS%", "\n  ".join(lines)))
    exe = tmp_path / "probe"
    subprocess.run([gcc, "-std=c99", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    out = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    assert int(out["dsa_fwd_args"]) == ctypes.sizeof(_lib.DsaFwdArgs)
    assert int(out["dsa_bwd_args"]) == ctypes.sizeof(_lib.DsaBwdArgs)
    for cname, st in (("dsa_fwd_args", _lib.DsaFwdArgs), ("dsa_bwd_args", _lib.DsaBwdArgs)):
        for fname, _ in st._fields_:
            assert int(out[f"{cname}.{fname}"]) == getattr(st, fname).offset, (cname, fname)


# --- torch.library ops ----------------------------------------------------------------
def _inputs(device="cpu", dtype=torch.bfloat16, B=2, L=64, H=2, D=64, A=16):
    mk = lambda *s: torch.randn(*s, device=device).to(dtype)
    q, k, v = mk(B, L, H, D), mk(B, L, H, D), mk(B, L, H, D)
    kr, qr = mk(H, 2 * A, D), mk(H, 2 * A, D)
    table = torch.arange(-(L - 1), L, dtype=torch.int32, device=device)
    return q, k, v, kr, qr, table


def test_ops_are_registered():
    assert hasattr(torch.ops.deberta_amd, "dsa_fwd")
    assert hasattr(torch.ops.deberta_amd, "dsa_bwd")


def test_cpu_tensors_fail_loudly():
    q, k, v, kr, qr, table = _inputs()
    with pytest.raises(NotImplementedError):
        torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, 16, 0.1)


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q, k, v, kr, qr, table = _inputs()
        out, lse, bias, _ = torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, 16, 0.1)
        assert out.shape == q.shape and out.dtype == q.dtype
        assert lse.shape == (2, 2, 64) and lse.dtype == torch.float32
        assert bias.shape == (2, 2, 128, 128) and bias.dtype == torch.float16
        g = torch.ops.deberta_amd.dsa_bwd(out, q, k, v, kr, qr, table, None, None, out, lse, bias, 16, 0.1)
        assert [t.shape for t in g] == [q.shape, k.shape, v.shape, (2, 32, 64), (2, 32, 64), (0,)]
        assert g[3].dtype == q.dtype
        # with the c2p term's query rows (qc, the carrier of p2p): their gradient
        g = torch.ops.deberta_amd.dsa_bwd(out, q, k, v, kr, qr, table, None, None, out, lse, bias, 16, 0.1, q)
        assert g[5].shape == q.shape
        b = torch.ops.deberta_amd.dsa_bias(q, k, kr, qr, table, 16, 0.1, None)
        assert b.shape == (2, 2, 64, 64) and b.dtype == q.dtype
        # with attention dropout: the keep bits come back as a fourth output,
        # followed (bf16, L = 64 > 2 A = 32) by O's rounding residual at the
        # next 256-byte boundary
        seed = torch.tensor([7], dtype=torch.int64)
        *_, bits = torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, 16, 0.1, True, None, 6554, seed)
        assert bits.shape == (2 * 2 * 4 * 2 * 64 * 4 + q.numel() * 2,) and bits.dtype == torch.uint8
        # neither without dropout and with L <= 2 A, nor without a saved term
        assert torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, 32, 0.1)[3].shape == (0,)
        assert torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, 16, 0.1, False)[3].shape == (0,)
        # the residual alone
        assert torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, 16, 0.1)[3].shape == (q.numel() * 2,)


def test_trace_forward_and_backward_with_fake_tensors():
    """make_fx in fake mode exercises the fake impls and the autograd
    registration together (the path torch.compile takes)."""
    from torch.fx.experimental.proxy_tensor import make_fx

    def f(q, k, v, kr, qr, table, dout):
        out, _, _, _ = torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, 16, 0.1)
        return torch.autograd.grad(out, (q, k, v, kr, qr), dout)

    q, k, v, kr, qr, table = _inputs()
    for t in (q, k, v, kr, qr):
        t.requires_grad_(True)
    gm = make_fx(f, tracing_mode="fake")(q, k, v, kr, qr, table, torch.randn_like(q))
    code = gm.code
    assert "deberta_amd.dsa_fwd" in code and "deberta_amd.dsa_bwd" in code


def test_python_validation():
    q, k, v, kr, qr, table = _inputs()
    with pytest.raises(ValueError, match="head dim"):
        ops._validate(q[..., :48], k[..., :48], v[..., :48], None, None, None, None, None, 16)
    with pytest.raises(ValueError, match=r"kr must be \[H"):
        ops._validate(q, k, v, kr[:, :10], None, table, None, None, 16)
    with pytest.raises(ValueError, match="rel_table"):
        ops._validate(q, k, v, kr, None, None, None, None, 16)
    with pytest.raises(TypeError, match="dtype"):
        ops._validate(q.half(), k.half(), v.half(), None, None, None, None, None, 16)


# --- host-side mirror of the reference interface -----------------------------------------
@pytest.mark.parametrize(
    "raw,canon",
    [
        ("dynamic", "dynamic"),
        ("default", "dynamic"),
        ("cached", "cached_bmm"),
        ("cache", "cached_bmm"),
        ("cached-bmm", "cached_bmm"),
        ("SAFE", "stable"),
        ("compile-safe", "stable"),
        ("hip", "fused"),
        ("fused", "fused"),
    ],
)
def test_attention_kernel_selector(raw, canon):
    assert normalize_attention_kernel(raw) == canon


def test_attention_kernel_selector_rejects():
    """test_smoke.py:2243 restated: the reference's error text."""
    with pytest.raises(ValueError, match="model.hf.attention_kernel must be one of"):
        normalize_attention_kernel("bad_kernel")


def test_pos_att_type_normaliser():
    assert normalize_pos_att_type("C2P|p2c") == ["c2p", "p2c"]
    assert normalize_pos_att_type("c2p, p2c") == ["c2p", "p2c"]
    assert normalize_pos_att_type(["p2c", "c2p"]) == ["p2c", "c2p"]
    assert normalize_pos_att_type(None) == []


def test_keep_mask_contract():
    with pytest.raises(TypeError):
        normalize_keep_mask([1])
    with pytest.raises(ValueError, match="Floating-point masks are ambiguous"):
        normalize_keep_mask(torch.ones(2))
    assert normalize_keep_mask(torch.tensor([3, 0])).tolist() == [True, False]
    assert get_attention_mask(torch.ones(2, 8, dtype=torch.long)).shape == (2, 1, 1, 8)
    assert get_attention_mask(torch.ones(2, 8, 8, dtype=torch.bool)).shape == (2, 1, 8, 8)
    assert get_attention_mask(torch.ones(2, 3, 8, 8, dtype=torch.bool)).shape == (2, 1, 8, 8)


def test_kernel_masks():
    keep = torch.tensor([[1, 1, 0, 1]], dtype=torch.bool)
    kk, pk = kernel_masks(keep[:, None, None, :], 3, 4, 4)
    assert pk is None and kk.shape == (3, 4) and kk.stride(0) == 0 and kk.dtype == torch.uint8
    assert kk[2].tolist() == [1, 1, 0, 1]
    dense = torch.ones(2, 1, 4, 4, dtype=torch.bool)
    kk, pk = kernel_masks(dense, 2, 4, 4)
    assert kk is None and pk.shape == (2, 4, 4) and pk.stride(-1) == 1
    assert kernel_masks(None, 2, 4, 4) == (None, None)
    with pytest.raises(ValueError, match="rank-4"):
        kernel_masks(torch.ones(2, 4, dtype=torch.bool), 2, 4, 4)


def test_pair_mask_rows_are_16_byte_aligned():
    """The kernels read pair-mask rows in 16-byte chunks: kernel_masks hands
    them rows whose stride is a multiple of 16 reaching round_up(L, 16),
    padding a copy with zeros when the input's rows do not."""
    g = torch.Generator().manual_seed(3)
    for L in (64, 700):
        dense = torch.rand(2, 1, L, L, generator=g) > 0.5
        kk, pk = kernel_masks(dense, 2, L, L)
        assert kk is None and pk.shape == (2, L, L) and pk.stride(-1) == 1
        assert pk.stride(-2) % 16 == 0 and pk.stride(-2) >= (L + 15) // 16 * 16 and pk.data_ptr() % 16 == 0
        assert torch.equal(pk.bool(), dense[:, 0])
        if L % 16:
            base = pk.as_strided((2, L, pk.stride(-2)), (pk.stride(0), pk.stride(1), 1))
            assert not base[:, :, L:].any()  # zero padding


def test_dense_document_masks_are_recognised():
    """dense_as_segments: a packed-document mask (reference form, pad rows
    keeping only their CLS edge) has segment ids with the kernels' rule,
    which then agrees with it on every live row; other masks have none."""
    from deberta_amd.masks import dense_as_segments

    ids = torch.tensor([[1, 1, 2, 2, 2, 3, 0, 0], [4, 4, 4, 4, 5, 5, 5, 0]])
    dense = build_doc_block_mask(ids)
    seg = dense_as_segments(dense)
    assert seg is not None and seg.dtype == torch.int32
    live = ids != 0
    rule = (seg[:, :, None] == seg[:, None, :]) & (seg[:, :, None] != 0)
    assert torch.equal(rule[live], dense[live]) and torch.equal(seg != 0, live)
    # interleaved segments are an equivalence too
    ids2 = torch.tensor([[1, 2, 1, 2, 3, 3, 1, 0]])
    assert dense_as_segments(build_doc_block_mask(ids2)) is not None
    # a causal mask is not one
    causal = torch.tril(torch.ones(8, 8, dtype=torch.bool))[None]
    assert dense_as_segments(causal) is None


def test_segment_mask_host_side():
    """SegmentMask is the ids form of the reference's packed-document mask:
    dense() is that mask, and the kernels get the ids as int32 [B, S]."""
    ids = torch.tensor([[1, 1, 2, 2, 2, 0], [5, 5, 5, 5, 0, 0]])
    m = SegmentMask(ids)
    assert m.shape == (2, 1, 6, 6)
    assert torch.equal(m.dense(), build_doc_block_mask(ids)[:, None])
    seg, pk = kernel_masks(m, 2, 6, 6)
    assert pk is None and seg.dtype == torch.int32 and seg.is_contiguous() and seg.tolist() == ids.tolist()
    # the kernels' rule (both ids equal and nonzero) gives the dense mask on
    # every live query row; pad rows are dead in both (the reference zeroes
    # their output), and only their CLS edge differs
    live = ids != 0
    rule = (ids[:, :, None] == ids[:, None, :]) & live[:, :, None]
    dense = m.dense()[:, 0]
    assert torch.equal(rule[live], dense[live])
    with pytest.raises(ValueError, match="does not match"):
        kernel_masks(m, 2, 6, 5)
    with pytest.raises(ValueError, match="rank-2"):
        SegmentMask(ids[0])
    with pytest.raises(ValueError, match="integer"):
        SegmentMask(ids.float())
    with pytest.raises(TypeError):
        SegmentMask([[1, 2]])


def test_mask_argument_errors(lib):
    a = _lib.DsaFwdArgs()
    a.B, a.H, a.Lq, a.Lk, a.D, a.dtype = 1, 1, 40000, 40000, 64, _lib.DSA_BF16
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p).value
    for f in ("q", "k", "v", "out", "lse"):
        setattr(a, f, p)
    a.seg = p
    assert lib.dsa_fwd(ctypes.byref(a), None) != 0
    assert "at most 32768 tokens" in _lib.last_error()
    a.key_keep = p
    assert lib.dsa_fwd(ctypes.byref(a), None) != 0
    assert "at most one of key_keep, pair_keep and seg" in _lib.last_error()
    a.key_keep, a.Lk = None, 100
    assert lib.dsa_fwd(ctypes.byref(a), None) != 0
    assert "Lq == Lk" in _lib.last_error()


@pytest.mark.parametrize("share", [False, True])
@pytest.mark.parametrize("types", ["c2p|p2c", "c2p", "p2c", "c2p|p2c|p2p"])
def test_module_layout_matches_the_reference_shape(share, types):
    """Same parameter names and shapes as the reference module (restated in
    the oracle), so reference state dicts load unchanged."""
    cfg = eager.make_config(hidden_size=64, num_attention_heads=4, share_att_key=share, pos_att_type=types)
    ours = DisentangledSelfAttention(cfg)
    ref = eager.EagerDisentangledSelfAttention(cfg)
    assert {k: v.shape for k, v in ours.state_dict().items()} == {k: v.shape for k, v in ref.state_dict().items()}
    ours.load_state_dict(ref.state_dict(), strict=True)
    assert ours.pos_ebd_size == 256 and ours.attn_kernel == "dynamic"


def test_module_rejects_bad_config_and_the_op_rejects_cpu():
    with pytest.raises(ValueError, match="divisible"):
        DisentangledSelfAttention(eager.make_config(hidden_size=30, num_attention_heads=4))
    with pytest.raises(ValueError, match="model.hf.attention_kernel must be one of"):
        DisentangledSelfAttention(eager.make_config(hf_attention_kernel="nope"))
    # the module runs CPU tensors on its torch path (tests/test_module_cpu.py);
    # the kernels' own entry, fused_attention, refuses them
    from deberta_amd.attention import fused_attention

    q = torch.randn(1, 8, 4, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        fused_attention(q, q, q, None, None, None, None, 1, 0.25)


def test_package_surface():
    for name in deberta_amd.__all__:
        assert hasattr(deberta_amd, name), name


def test_segment_cache_is_keyed_by_identity_and_keeps_the_mask_batch():
    """The dense-mask recognition cache is looked up twice with the same mask
    object (layer 2 of an encoder, the next step): identity-keyed, so the
    lookup never compares tensors elementwise.  A broadcast (1, 1, S, S)
    mask keeps one row of ids, expanded to each call's batch."""
    from deberta_amd.masks import _SEGMENTS_OF, _segments_cached

    ids = torch.tensor([[1, 1, 2, 2, 2, 3, 0, 0]])
    mask = build_doc_block_mask(ids)[:, None]
    pk = mask.view(torch.uint8)[:, 0]
    first = _segments_cached(mask, pk)
    second = _segments_cached(mask, pk)
    assert first is second and first.shape == (1, 8)
    other = mask.clone()
    assert _segments_cached(other, other.view(torch.uint8)[:, 0]) is not first
    other[0, 0, 0, 0] = False  # a new version is checked again
    assert _segments_cached(other, other.view(torch.uint8)[:, 0]) is None
    assert mask in _SEGMENTS_OF and other in _SEGMENTS_OF


def test_mask_shapes_are_checked_before_launch():
    """ops._validate refuses masks whose extent differs from (B, Lk) /
    (B, Lq, Lk): the kernels would read them out of bounds."""
    q, k, v, kr, qr, table = _inputs(B=2, L=64)
    good = torch.ones(2, 64, dtype=torch.uint8)
    ops._validate(q, k, v, kr, qr, table, good, None, 16)
    ops._validate(q, k, v, kr, qr, table, good[:1].expand(2, 64), None, 16)  # batch stride 0
    with pytest.raises(ValueError, match=r"key_keep / segment ids must be \[B=2, Lk=64\]"):
        ops._validate(q, k, v, kr, qr, table, good[:1], None, 16)
    with pytest.raises(ValueError, match="key_keep / segment ids"):
        ops._validate(q, k, v, kr, qr, table, torch.ones(2, 63, dtype=torch.int32), None, 16)
    with pytest.raises(TypeError, match="key_keep must be uint8"):
        ops._validate(q, k, v, kr, qr, table, good.float(), None, 16)
    with pytest.raises(ValueError, match=r"pair_keep must be \[B=2, Lq=64, Lk=64\]"):
        ops._validate(q, k, v, kr, qr, table, None, torch.ones(1, 64, 64, dtype=torch.uint8), 16)


def test_deterministic_mode_alerts_on_table_gradients():
    """torch.use_deterministic_algorithms(True) refuses the backward with
    relative tables (dkr / dqr are summed with fp32 atomics); warn_only
    warns.  Checked before any device work."""
    prev, prev_warn = torch.are_deterministic_algorithms_enabled(), torch.is_deterministic_algorithms_warn_only_enabled()
    try:
        torch.use_deterministic_algorithms(True)
        with pytest.raises(RuntimeError, match="deterministic implementation"):
            ops._alert_nondeterministic_tables()
        torch.use_deterministic_algorithms(True, warn_only=True)
        with pytest.warns(UserWarning, match="deterministic implementation"):
            ops._alert_nondeterministic_tables()
        torch.use_deterministic_algorithms(False)
        ops._alert_nondeterministic_tables()
    finally:
        torch.use_deterministic_algorithms(prev, warn_only=prev_warn)


# --- the fused row kernels around the attention (include/dsa_block.h) ---------------------
BLOCK_HEADER = ROOT / "include" / "dsa_block.h"


def test_block_header_matches_the_exports(lib):
    text = re.sub(r"/\*.*?\*/", "", BLOCK_HEADER.read_text(), flags=re.S)
    declared = sorted(set(re.findall(r"\b(dsa_[a-z_]+)\s*\([^;{]*\)\s*;", text)))
    assert declared == sorted(_lib.BLOCK_EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_block_structs_match_the_c_header(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    structs = (("dsa_ln_args", _lib.DsaLnArgs), ("dsa_gelu_args", _lib.DsaGeluArgs), ("dsa_rtd_args", _lib.DsaRtdArgs))
    lines = [f'printf("{c} %zu\\n", sizeof({c}));' for c, _ in structs]
    for cname, st in structs:
        for fname, _ in st._fields_:
            lines.append(f"F({cname}, {fname})")
    src = tmp_path / "probe.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "dsa_block.h"\n'
        '#define F(s, f) printf(#s "." #f " %zu\\n", offsetof(s, f));\n'
        "int main(void) {\n  " + "\n  ".join(lines) + "\n  return 0;\n}\n"
    )
    exe = tmp_path / "probe"
    subprocess.run([gcc, "-std=c99", "-I", str(BLOCK_HEADER.parent), str(src), "-o", str(exe)], check=True)
    out = dict(l.rsplit(" ", 1) for l in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    for cname, st in structs:
        assert int(out[cname]) == ctypes.sizeof(st), cname
        for fname, _ in st._fields_:
            assert int(out[f"{cname}.{fname}"]) == getattr(st, fname).offset, (cname, fname)


def test_block_argument_errors(lib):
    a = _lib.DsaLnArgs()
    assert lib.dsa_add_ln_fwd(ctypes.byref(a), None) != 0
    assert "dsa_add_ln" in _lib.last_error()
    a.N, a.C = 4, 4098
    assert lib.dsa_add_ln_fwd(ctypes.byref(a), None) != 0
    assert "multiple of 4 in [4, 2048]" in _lib.last_error()
    r = _lib.DsaRtdArgs()
    r.N, r.C = 8, 64
    assert lib.dsa_rtd_loss_fwd(ctypes.byref(r), None) != 0
    assert "x, w and labels are required" in _lib.last_error()
    assert lib.dsa_block_workspace_bytes(_lib.DSA_BLOCK_LN, 8192, 768) >= 256 * 3 * 768 * 4


def test_block_ops_fake_shapes_and_cpu_refusal():
    from torch._subclasses.fake_tensor import FakeTensorMode

    import deberta_amd.blocks  # noqa: F401  (registers the ops)

    with FakeTensorMode():
        x = torch.randn(2, 8, 64, dtype=torch.bfloat16)
        w, b = torch.randn(64), torch.randn(64)
        y, mean, rstd = torch.ops.deberta_amd.add_ln(x, b, x.float(), w, b, 1e-7, torch.float32)
        assert y.shape == x.shape and y.dtype == torch.float32 and mean.shape == (16,)
        assert torch.ops.deberta_amd.bias_gelu(x, b.bfloat16()).shape == x.shape
        loss, logits, denom = torch.ops.deberta_amd.rtd_loss(x, w, b[:1], torch.ones(2, 8), None)
        assert loss.shape == () and logits.shape == (2, 8)
    with pytest.raises(NotImplementedError):
        torch.ops.deberta_amd.bias_gelu(torch.randn(2, 64), None)


def test_fused_blocks_take_the_reference_state_dicts():
    from deberta_amd import FusedIntermediate, FusedOutput, FusedRTDHead, FusedSelfOutput, RelativeEmbeddings
    from oracle import blocks as ob

    cfg = eager.make_config(hidden_size=64, num_attention_heads=4, intermediate_size=256, layer_norm_eps=1e-7)
    for ours, ref in (
        (FusedSelfOutput(cfg), ob.OutputResidualNorm(cfg)),
        (FusedOutput(cfg), ob.OutputResidualNorm(cfg, in_features=256)),
        (FusedIntermediate(cfg), ob.Intermediate(cfg)),
        (FusedRTDHead(cfg), ob.RTDHead(cfg)),
        (RelativeEmbeddings(cfg), ob.RelativeEmbeddings(cfg)),
    ):
        assert {k: v.shape for k, v in ours.state_dict().items()} == {k: v.shape for k, v in ref.state_dict().items()}
        ours.load_state_dict(ref.state_dict(), strict=True)
    with pytest.raises(NotImplementedError, match="gelu"):
        FusedIntermediate(eager.make_config(hidden_size=64, intermediate_size=256, hidden_act="relu"))


def test_per_head_masks_become_head_strided_pair_masks():
    """A (B, H, S, S) keep mask reaches the kernels as a [B, H, S, S] byte
    view whose batch, head and row strides are multiples of 16 bytes (rows
    padded to 16 when they are not); (B, H, 1, S) repeats one row per head
    for every query; a head count other than 1 or H is refused."""
    B, H, S = 2, 3, 24
    m = torch.rand(B, H, S, S) < 0.5
    kk, pk = kernel_masks(m, B, S, S, heads=H)
    assert kk is None and pk.shape == (B, H, S, S) and pk.dtype == torch.uint8
    assert all(s % 16 == 0 for s in pk.stride()[:3]) and pk.stride(-1) == 1
    assert torch.equal(pk.bool(), m)
    m2 = torch.rand(1, H, 1, 32) < 0.5
    _, pk2 = kernel_masks(m2, B, 32, 32, heads=H)
    assert pk2.shape == (B, H, 32, 32) and pk2.stride(2) == 0 and pk2.stride(0) == 0
    assert torch.equal(pk2[1, 2, 17].bool(), m2[0, 2, 0])
    with pytest.raises(ValueError, match="head dim"):
        kernel_masks(torch.ones(B, 2, S, S, dtype=torch.bool), B, S, S, heads=H)
    q, k, v, _, _, _ = _inputs(B=B, L=S, H=H)
    ops._validate(q, k, v, None, None, None, None, pk, 16)
    args = ops._fill_fwd_args(q, k, v, None, None, None, None, pk, q, torch.empty(1), 16, 0.1)
    assert args.pair_keep_stride_h == pk.stride(1) and tuple(args.pair_keep_strides) == (pk.stride(0), pk.stride(2))


def test_ops_refuse_graph_capture(monkeypatch):
    """Every op implementation refuses to launch while the current stream is
    capturing a CUDA/HIP graph (the query is patched: no graph is captured
    here), before it validates or allocates anything."""
    import deberta_amd.blocks as blocks
    from deberta_amd import ops

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    q, k, v, kr, qr, table = _inputs()
    calls = [
        lambda: ops._dsa_fwd_impl(q, k, v, kr, qr, table, None, None, 16, 0.1),
        lambda: ops._dsa_bwd_impl(q, q, k, v, kr, qr, table, None, None, q, q, q, 16, 0.1),
        lambda: ops._dsa_bias_impl(q, k, kr, qr, table, 16, 0.1),
        lambda: ops._dsa_fwd_packed_impl(torch.stack([q, k, v], 2), kr, qr, table, None, None, 16, 0.1),
        lambda: blocks._add_ln_impl(q, None, None, q, q, 1e-7, q.dtype),
        lambda: blocks._add_ln_bwd_impl(q, q, None, None, q, q, q, q.dtype),
        lambda: blocks._bias_gelu_impl(q, None),
        lambda: blocks._bias_gelu_bwd_impl(q, q, None),
        lambda: blocks._rtd_loss_impl(q, q, None, q, None),
        lambda: blocks._rtd_loss_bwd_impl(q, q, q, None, q, None, q, q),
    ]
    for call in calls:
        with pytest.raises(RuntimeError, match="capturing a CUDA/HIP graph"):
            call()


def test_dropout_argument_errors(lib):
    """Attention dropout's threshold is checked before any device work, and
    the package's helpers map a probability to the kernels' threshold and
    refuse a missing or malformed seed."""
    a = _lib.DsaFwdArgs()
    a.B, a.H, a.Lq, a.Lk, a.D, a.dtype = 1, 1, 8, 8, 64, _lib.DSA_BF16
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p).value
    for f in ("q", "k", "v", "out", "lse"):
        setattr(a, f, p)
    a.dropout_threshold = 65536
    assert lib.dsa_fwd(ctypes.byref(a), None) != 0
    assert "dropout_threshold must be in [0, 65535]" in _lib.last_error()
    assert ops.dropout_threshold(0.1) == 6554 and ops.dropout_threshold(0.5) == 32768
    assert ops.dropout_threshold(1e-6) == 0 and ops.dropout_threshold(1 - 1e-6) == 65536
    with pytest.raises(ValueError, match="dropout threshold"):
        ops._check_threshold(70000)
    with pytest.raises(ValueError, match="dropout_seed"):
        ops._seed_value(None, 6554)
    with pytest.raises(ValueError, match="dropout_seed"):
        ops._seed_value(torch.tensor([1, 2]), 6554)
    assert ops._seed_value(None, 0) == 0
    assert ops._seed_value(torch.tensor([-1]), 6554) == (1 << 64) - 1
    s = ops.draw_dropout_seed()
    assert s.dtype == torch.int64 and s.numel() == 1 and s.device.type == "cpu" and 0 <= int(s) < (1 << 62)
    torch.manual_seed(5)
    s1 = ops.draw_dropout_seed()
    torch.manual_seed(5)
    assert torch.equal(s1, ops.draw_dropout_seed())


def test_dropout_bytes_match_the_library(lib):
    """The package's size of the keep bits (fake implementations use it)
    equals the library's dsa_fwd_dropout_bytes."""
    for B, H, Lq, Lk in ((1, 1, 1, 1), (2, 3, 200, 200), (4, 12, 4096, 4096), (2, 2, 64, 300)):
        a = _lib.DsaFwdArgs()
        a.B, a.H, a.Lq, a.Lk, a.D, a.dtype = B, H, Lq, Lk, 64, _lib.DSA_BF16
        a.dropout_threshold = 6554
        q = torch.empty(B, Lq, H, 64, device="meta")
        k = torch.empty(B, Lk, H, 64, device="meta")
        assert lib.dsa_fwd_dropout_bytes(ctypes.byref(a)) == ops.dropout_bytes(q, k, 6554)
        a.dropout_threshold = 0
        assert lib.dsa_fwd_dropout_bytes(ctypes.byref(a)) == 0 == ops.dropout_bytes(q, k, 0)
