"""The module under torch.compile's CUDA-graph mode ``reduce-overhead`` (one
of the reference's ``compile.mode`` choices, src/deberta/config.py:54-59;
``max-autotune`` captures the same way and adds GEMM autotuning), with
``cudagraph_mark_step_begin`` per step as training/compile.py:115-123
does.

The attention ops are tagged CUDA-graph unsafe (deberta_amd/ops.py), so
inductor runs them between captured graph partitions rather than capturing
them.  Every replay must equal the eager module: output and every gradient
to 2e-2 of their scale (the compiled projections may round differently),
over several steps in a row with eager work and synchronisations between
them.  The key-projection bias's gradient (exactly zero: softmax ignores
a shift of every key) is compared on its weight gradient's scale.
"""

from __future__ import annotations

import sys

import pytest
import torch

from deberta_amd import DisentangledSelfAttention
from tests._modules import _errors

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


def _config():
    return type(
        "Cfg",
        (),
        dict(hidden_size=256, num_attention_heads=4, share_att_key=True, pos_att_type="p2c|c2p",
             relative_attention=True, position_buckets=256, max_relative_positions=-1,
             max_position_embeddings=512, hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0),
    )()


@pytest.mark.parametrize("mode", ["reduce-overhead"])
def test_cudagraph_compile_modes_match_eager(mode, gpu):
    torch._dynamo.reset()
    torch.manual_seed(0)
    layer = DisentangledSelfAttention(_config()).to(gpu, torch.bfloat16)
    with torch.no_grad():
        for n, p in layer.named_parameters():
            p.copy_(torch.randn_like(p) * 0.02 if n.endswith("weight") else torch.zeros_like(p))
    g = torch.Generator().manual_seed(57)
    x0 = torch.randn(2, 256, 256, generator=g).to(gpu, torch.bfloat16)
    rel0 = (torch.randn(512, 256, generator=g) * 0.02).to(gpu, torch.bfloat16)
    dout = torch.randn(2, 256, 256, generator=g).to(gpu, torch.bfloat16)
    params = list(layer.parameters())

    def step(module):
        x = x0.clone().requires_grad_(True)
        rel = rel0.clone().requires_grad_(True)
        out, _ = module(x, None, rel_embeddings=rel)
        grads = torch.autograd.grad(out, [x, rel] + params, dout)
        return [out.detach().float().clone()] + [t.float().clone() for t in grads]

    ref = step(layer)
    compiled = torch.compile(layer, mode=mode, dynamic=False)
    names = ["out", "dx", "drel"] + [f"d{n}" for n, _ in layer.named_parameters()]
    for r in range(4):
        torch.compiler.cudagraph_mark_step_begin()
        got = step(compiled)
        y = torch.randn(512, 512, device=gpu)
        (y @ y).sum().item()  # eager work and a synchronisation between the steps
        torch.cuda.synchronize(gpu)
        errs = _errors(dict(zip(names, ref)), dict(zip(names, got)))
        _say(f"[{mode}] step {r}: {errs}")
        bad = {n: e for n, e in errs.items() if not e <= 2e-2}
        assert not bad, f"{mode} step {r}: {bad}"
