"""Ordered microbatch execution of one logical batch (the streamed runtime).

Restates solution/shape14/executor.py:12-49 of the reference: validate the
microbatch, run ordered slices ``value[start:end]`` (with the matching mask
slice) through ``forward_chunk`` and assemble the logical output.

Addition for HBM-resident long sequences: with ``write_into_output=True`` the
output is allocated once up front (same shape and dtype as the input) and
``forward_chunk`` receives the destination slice as a third argument, so a
chunk whose last kernel writes straight into that slice needs no
device-to-device copy (the reference copies every chunk, executor.py:46).
A chunk that returns another tensor is still copied.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

ChunkForward = Callable[..., torch.Tensor]


def _validate(value: torch.Tensor, valid_token_mask: torch.Tensor | None, microbatch_size: object) -> int:
    if (
        isinstance(microbatch_size, bool)
        or not isinstance(microbatch_size, int)
        or microbatch_size <= 0
    ):
        raise ValueError("microbatch_size must be a positive integer")
    batch_size = value.shape[0]
    if batch_size <= 0:
        raise ValueError("streamed execution requires a non-empty batch")
    if batch_size % microbatch_size:
        raise ValueError("microbatch_size must divide the batch size")
    if valid_token_mask is not None and valid_token_mask.shape[0] != batch_size:
        raise ValueError("valid_token_mask batch dimension must match the input")
    return batch_size


def execute_streamed(
    value: torch.Tensor,
    valid_token_mask: torch.Tensor | None,
    *,
    microbatch_size: int,
    forward_chunk: ChunkForward,
    write_into_output: bool = False,
) -> torch.Tensor:
    """Execute one logical batch as ordered microbatches."""

    batch_size = _validate(value, valid_token_mask, microbatch_size)
    output: torch.Tensor | None = torch.empty_like(value) if write_into_output else None
    for start in range(0, batch_size, microbatch_size):
        end = start + microbatch_size
        mask_slice = None if valid_token_mask is None else valid_token_mask[start:end]
        if write_into_output:
            assert output is not None
            destination = output[start:end]
            chunk = forward_chunk(value[start:end], mask_slice, destination)
            if chunk.data_ptr() != destination.data_ptr() or chunk.shape != destination.shape:
                destination.copy_(chunk)
            continue
        chunk = forward_chunk(value[start:end], mask_slice)
        if output is None:
            output = torch.empty((batch_size, *chunk.shape[1:]), dtype=chunk.dtype, device=chunk.device)
        output[start:end].copy_(chunk)
    assert output is not None
    return output


__all__ = ["execute_streamed"]
