"""Eager-mode dispatch of the package's custom ops.

A ``torch.library`` custom op costs tens of microseconds of host time per
call (dispatcher round trips, default filling, the autograd wrapper around
the Python kernel), and an encoder step makes hundreds of such calls, so a
many-layer step becomes bound by the host.  In plain eager mode the package
therefore runs each op's implementation directly inside a
``torch.autograd.Function`` built from the same setup-context and backward
functions the op registers with ``register_autograd``.  Under
``torch.compile``, under an active dispatch mode (fake tensors, tracing) or
for a tensor subclass, calls go through ``torch.ops`` so that tracing sees
the op and its fake implementation.  Both paths launch the same kernels.
"""

from __future__ import annotations

from typing import Any, Callable

import torch

_dispatch_depth = torch._C._len_torch_dispatch_stack
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def eager(t: torch.Tensor) -> bool:
    """True when a call with main input ``t`` may bypass ``torch.ops``."""
    # is_compiling() first: dynamo folds it to True while tracing, and the
    # dispatch-stack query after it (a C function dynamo does not trace)
    # would otherwise break the graph
    return not torch.compiler.is_compiling() and type(t) is torch.Tensor and _dispatch_depth() == 0


def refuse_capture(what: str) -> None:
    """Raise when the current stream is capturing a CUDA/HIP graph.  Capturing
    the library's launches (torch.cuda.graph around the attention op) ended
    in a host fault inside the runtime's capture end, whose cause is not
    known, so the ops refuse to run under capture.  torch.compile's
    CUDA-graph modes run them between the captured partitions instead (the
    ops are tagged cudagraph_unsafe)."""
    if torch.cuda.is_current_stream_capturing():
        raise RuntimeError(
            f"{what}: the current stream is capturing a CUDA/HIP graph; the fused kernels are not supported "
            "under graph capture (torch.compile's reduce-overhead / max-autotune modes run them outside the "
            "captured partitions)"
        )


def stream_ptr(t: torch.Tensor) -> int:
    """The raw handle of the current HIP stream of ``t``'s device."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def function(
    name: str,
    impl: Callable[..., Any],
    setup_context: Callable[[Any, tuple, Any], None],
    backward: Callable[..., Any],
) -> type:
    """A ``torch.autograd.Function`` whose forward is ``impl`` followed by
    ``setup_context(ctx, inputs, output)`` and whose backward is
    ``backward``; ``ctx.eager`` is set so the backward calls the
    implementations of its ops directly too."""

    def forward(ctx, *inputs):
        output = impl(*inputs)
        ctx.eager = True
        setup_context(ctx, inputs, output)
        return output

    return type(name, (torch.autograd.Function,), {"forward": staticmethod(forward), "backward": staticmethod(backward)})


def on_eager(ctx: Any, op: Any, impl: Callable[..., Any]) -> Callable[..., Any]:
    """The callable a registered backward uses for one of its ops: the raw
    implementation in eager mode, the op otherwise."""
    return impl if getattr(ctx, "eager", False) else op
