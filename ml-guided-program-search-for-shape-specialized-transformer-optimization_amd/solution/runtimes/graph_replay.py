"""Graph replay of one fixed execution plan (the ``cuda_graph`` runtime).

Same contract as the reference's solution/runtimes/cuda_graph.py:11-141: one
static input signature per model, captured once on a side stream after
warm-up passes; every call copies the input (and mask) into the captured
buffers, replays, and returns an output the caller owns.  On ROCm
``torch.cuda.CUDAGraph`` records a HIP graph; the HIP kernels of this build
launch on the current stream, allocate only through torch's caching allocator
(the graph's private pool) and never synchronize, so they are capturable.

``reuse_unchanged_input`` skips the staging copy when the same input tensor
is passed again unmodified (its autograd version counter is unchanged).
"""

from __future__ import annotations

import weakref
from collections.abc import Callable

import torch

Forward = Callable[[torch.Tensor, torch.Tensor | None], torch.Tensor]


def _signature(value: torch.Tensor, mask: torch.Tensor | None) -> tuple[object, ...]:
    mask_part = None
    if mask is not None:
        mask_part = (mask.device, mask.dtype, tuple(mask.shape), tuple(mask.stride()))
    return (value.device, value.dtype, tuple(value.shape), tuple(value.stride()), mask_part)


def _version(value: torch.Tensor) -> int | None:
    try:
        version = value._version
    except RuntimeError:  # inference tensors have no version counter
        return None
    return version if isinstance(version, int) else None


class GraphReplay:
    """Capture one static signature of ``forward`` and replay it."""

    WARMUP_PASSES = 3

    def __init__(self, *, reuse_unchanged_input: bool = False) -> None:
        self.reuse_unchanged_input = reuse_unchanged_input
        self._signature: tuple[object, ...] | None = None
        self._graph: torch.cuda.CUDAGraph | None = None
        self._input: torch.Tensor | None = None
        self._mask: torch.Tensor | None = None
        self._output: torch.Tensor | None = None
        self._staged: weakref.ReferenceType[torch.Tensor] | None = None
        self._staged_version: int | None = None

    @property
    def captured(self) -> bool:
        return self._graph is not None

    def _capture(self, forward: Forward, value: torch.Tensor, mask: torch.Tensor | None) -> None:
        static_input = value.detach().clone()
        static_mask = None if mask is None else mask.detach().clone()
        current = torch.cuda.current_stream(value.device)
        side = torch.cuda.Stream(device=value.device)  # default priority
        side.wait_stream(current)
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(self.WARMUP_PASSES):  # library handles and workspaces exist before capture
                forward(static_input, static_mask)
        current.wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(graph, stream=side):
            static_output = forward(static_input, static_mask)
        current.wait_stream(side)
        # Published only after warm-up and capture both succeeded.
        self._signature = _signature(value, mask)
        self._graph = graph
        self._input, self._mask, self._output = static_input, static_mask, static_output
        self._staged = None
        self._staged_version = None

    def _input_is_staged(self, value: torch.Tensor) -> bool:
        if not self.reuse_unchanged_input or self._staged is None:
            return False
        version = _version(value)
        return version is not None and self._staged() is value and self._staged_version == version

    def run(self, forward: Forward, value: torch.Tensor, mask: torch.Tensor | None) -> torch.Tensor:
        signature = _signature(value, mask)
        if self._graph is not None and signature != self._signature:
            raise RuntimeError(
                "graph replay supports one static input signature per model; "
                "reconfigure the model for a different signature"
            )
        if self._graph is None:
            self._capture(forward, value, mask)
        assert self._graph is not None and self._input is not None and self._output is not None
        if not self._input_is_staged(value):
            self._input.copy_(value)
            version = _version(value)
            if self.reuse_unchanged_input and version is not None:
                self._staged, self._staged_version = weakref.ref(value), version
            else:
                self._staged, self._staged_version = None, None
        if mask is not None:
            assert self._mask is not None
            self._mask.copy_(mask)
        self._graph.replay()
        return self._output.clone()


__all__ = ["GraphReplay"]
