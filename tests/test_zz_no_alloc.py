"""sah_causal_attention_bsd_static_workspace, the attention entry point that
allocates nothing (its workspace is a static device array), against
sah_causal_attention_bsd with a caller-provided workspace.  Where the
workspace (norm tables and fp16 scaled keys from 4096 keys on, and the
key-major copy of a seq-contiguous V^T) fits the array, both run the same
kernels.  Where it does not, the static entry runs the call in chunks of
heads of one batch row whose workspace fits; heads are independent and each
takes its path from its own tables, so the outputs must be bitwise equal in
both cases.  Each case makes two calls in a row, the second on a smaller
input, so the second reads the array the first left behind.  Both entry
points are called through the C ABI (ctypes)."""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

HEADER = Path(__file__).resolve().parents[1] / "include" / "shape_aware_hip.h"


def _inputs(batch, heads, seq, dtype, seed, seq_major_v, device):
    generator = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(batch, heads, seq, 64, generator=generator).to(dtype) for _ in range(3))
    q, k = q.to(device), k.to(device)
    if not seq_major_v:
        return q, k, v.to(device)
    pad = -(-seq // 8) * 8
    vt = torch.zeros(batch, heads, 64, pad, dtype=dtype)
    vt[..., :seq] = v.transpose(-2, -1)
    # [B, H, S, 64] view with seq stride 1, made on the device buffer
    return q, k, vt.to(device)[..., :seq].transpose(-2, -1)


def _call(library, static, q, k, v, launch, scale, dtype_code, stream):
    batch, heads, seq, _ = q.shape
    out = torch.full((batch, seq, heads * 64), float("nan"), dtype=q.dtype, device=q.device)
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), batch, heads, seq, 64,
            *q.stride()[:3], *k.stride()[:3], *v.stride(), out.stride(0), out.stride(1),
            scale, dtype_code, *launch]
    if static:
        status = library.sah_causal_attention_bsd_static_workspace(*args, stream)
    else:
        need = library.sah_causal_attention_workspace_bytes(
            batch, heads, seq, 64, v.stride(2), v.stride(3), dtype_code)
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
        status = library.sah_causal_attention_bsd(*args, workspace.data_ptr() if need else None, need, stream)
    assert status == 0, library.sah_last_error()
    return out


CASES = [
    # (dtype, seq-contiguous V, launch, first (B, H, S), second smaller (B, H, S))
    (torch.bfloat16, False, (256, 64, 8, 2), (2, 16, 2048), (1, 4, 700)),
    (torch.bfloat16, True, (256, 64, 8, 2), (1, 8, 20000), (1, 2, 16400)),
    (torch.float16, False, (128, 64, 4, 2), (2, 4, 1500), (1, 3, 129)),
    (torch.bfloat16, False, (128, 64, 4, 3), (1, 4, 17000), (1, 2, 333)),
]

# Calls whose workspace exceeds the static array: the static entry runs them
# in head chunks.  (dtype, seq-contiguous V, launch, first, second smaller)
CHUNKED_CASES = [
    # BASELINE C4's attention (B16 H32 S4096): the scaled keys alone are
    # 268 MB; one batch row (32 heads, 16.8 MB) fits.
    (torch.bfloat16, False, (256, 64, 8, 2), (16, 32, 4096), (2, 16, 4500)),
    # the same with V seq-contiguous: scaled keys and the key-major V copy
    (torch.bfloat16, True, (256, 64, 8, 2), (16, 32, 4096), (2, 16, 4500)),
    # one row of 16 heads just over 64 MiB with the V copy: chunks of 15 + 1
    (torch.bfloat16, True, (256, 64, 8, 2), (1, 16, 16384), (1, 8, 5000)),
    # a long sequence: 12.8 MB of scaled keys per head, chunks of 4 heads
    (torch.float16, False, (128, 64, 4, 2), (1, 16, 100000), (1, 3, 70000)),
]


def test_header_states_the_static_workspace_size():
    from solution.kernels.hip import _library

    match = re.search(r"#define SAH_ATTENTION_STATIC_WORKSPACE_BYTES \((\d+)ull << (\d+)\)", HEADER.read_text())
    assert match and int(match.group(1)) << int(match.group(2)) == _library.ATTENTION_STATIC_WORKSPACE_BYTES


@pytest.mark.parametrize("dtype,seq_major_v,launch,first,second", CASES)
def test_static_workspace_matches_caller_workspace(gpu_device, dtype, seq_major_v, launch, first, second):
    from solution.kernels.hip._library import dtype_code, load_library, stream_handle

    library = load_library()
    stream = stream_handle(gpu_device)
    for index, shape in enumerate((first, second)):
        print(f"static workspace dtype={dtype} seq_major_v={seq_major_v} launch={launch} "
              f"call={index} shape={shape}", flush=True)
        q, k, v = _inputs(*shape, dtype, 100 + index, seq_major_v, gpu_device)
        assert (v.stride(2) == 1) == seq_major_v
        want = _call(library, False, q, k, v, launch, 0.125, dtype_code(dtype), stream)
        got = _call(library, True, q, k, v, launch, 0.125, dtype_code(dtype), stream)
        torch.cuda.synchronize(gpu_device)
        assert bool(torch.isfinite(got).all())
        assert torch.equal(got, want), f"call {index} {shape}: outputs differ"


@pytest.mark.parametrize("dtype,seq_major_v,launch,first,second", CHUNKED_CASES)
def test_static_workspace_runs_head_chunks_when_the_call_does_not_fit(
    gpu_device, dtype, seq_major_v, launch, first, second
):
    from solution.kernels.hip._library import ATTENTION_STATIC_WORKSPACE_BYTES, dtype_code, load_library, stream_handle

    library = load_library()
    stream = stream_handle(gpu_device)
    batch, heads, seq = first
    v_stride_s, v_stride_d = (1, seq) if seq_major_v else (64, 1)
    need = library.sah_causal_attention_workspace_bytes(
        batch, heads, seq, 64, v_stride_s, v_stride_d, dtype_code(dtype))
    assert need > ATTENTION_STATIC_WORKSPACE_BYTES
    for index, shape in enumerate((first, second)):
        print(f"static workspace head chunks dtype={dtype} seq_major_v={seq_major_v} launch={launch} "
              f"call={index} shape={shape}", flush=True)
        q, k, v = _inputs(*shape, dtype, 200 + index, seq_major_v, gpu_device)
        assert (v.stride(2) == 1) == seq_major_v
        want = _call(library, False, q, k, v, launch, 0.125, dtype_code(dtype), stream)
        got = _call(library, True, q, k, v, launch, 0.125, dtype_code(dtype), stream)
        torch.cuda.synchronize(gpu_device)
        assert bool(torch.isfinite(got).all())
        assert torch.equal(got, want), f"call {index} {shape}: outputs differ"
        del q, k, v, want, got


def test_requests_beyond_the_static_workspace_are_rejected_before_launch(gpu_device):
    from solution.kernels.hip._library import load_library, stream_handle
    from solution.kernels.hip import _library

    library = load_library()
    # one head whose key-major V copy alone (600000 keys x 128 bytes) is
    # above the array: no chunk fits
    batch, heads, seq = 1, 1, 600000
    need = library.sah_causal_attention_workspace_bytes(batch, heads, seq, 64, 1, seq, 2)
    assert need > _library.ATTENTION_STATIC_WORKSPACE_BYTES
    # full-size buffers, so that no access could leave them even if a launch happened
    q = torch.zeros(batch, heads, seq, 64, dtype=torch.bfloat16, device=gpu_device)
    value = torch.zeros(batch, heads, 64, seq, dtype=torch.bfloat16, device=gpu_device).transpose(-1, -2)
    out = torch.empty(batch, seq, heads * 64, dtype=torch.bfloat16, device=gpu_device)
    status = library.sah_causal_attention_bsd_static_workspace(
        q.data_ptr(), q.data_ptr(), value.data_ptr(), out.data_ptr(), batch, heads, seq, 64,
        *q.stride()[:3], *q.stride()[:3], *value.stride(), out.stride(0), out.stride(1),
        0.125, 2, 256, 64, 8, 2, stream_handle(gpu_device))
    assert status == _library.SAH_ERR_WORKSPACE
    assert b"static workspace" in library.sah_last_error()
