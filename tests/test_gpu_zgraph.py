"""The fused forward + backward under HIP graph capture.

Every launch of the library goes on the caller's stream.  Replays must
equal the eager results exactly (dKr and dQr up to the order of their fp32
atomic additions), several times in a row, with eager work and
synchronisations between the replays.
"""

from __future__ import annotations

import math
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.skip(
    reason="graph capture of the op ended in a host segmentation fault inside "
    "torch.cuda.graph's capture_end (hipStreamEndCapture / instantiation), with "
    "and without the side-stream fork/join an earlier backward had; cause not yet shown, so "
    "the case stays off the GPU"
)
def test_graph_capture_replays_match_eager(gpu):
    from deberta_amd.relpos import relative_offset_table

    B, L, H, D, A = 2, 256, 4, 64, 256
    g = torch.Generator().manual_seed(21)
    mk = lambda *s: torch.randn(*s, generator=g).to(gpu, torch.bfloat16)
    q, k, v = (mk(B, L, H, D).requires_grad_(True) for _ in range(3))
    kr, qr = (mk(H, 2 * A, D).requires_grad_(True) for _ in range(2))
    dout = mk(B, L, H, D)
    table = relative_offset_table(L, L, bucket_size=256, max_position=512, device=gpu)
    scale = 1 / math.sqrt(D * 3)
    leaves = [q, k, v, kr, qr]

    def step():
        out, _, _, _ = torch.ops.deberta_amd.dsa_fwd(q, k, v, kr, qr, table, None, None, A, scale)
        return [out] + list(torch.autograd.grad(out, leaves, dout))

    ref = [t.clone() for t in step()]  # eager
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize(gpu)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for r in range(3):
        x = torch.randn(512, 512, device=gpu)
        (x @ x).sum().item()  # eager work and a synchronisation between replays
        graph.replay()
        torch.cuda.synchronize(gpu)
        print(f"[graph] replay {r}", file=sys.stderr, flush=True)
        for name, a, b in zip(["out", "dq", "dk", "dv", "dkr", "dqr"], outs, ref):
            if name in ("dkr", "dqr"):  # fp32 atomics: equal up to the order of the additions
                err = (a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30)
                assert err <= 1e-2, f"replay {r}: {name} differs from eager ({float(err):.3e})"
            else:
                assert torch.equal(a, b), f"replay {r}: {name} differs from eager"
