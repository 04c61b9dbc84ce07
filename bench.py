#!/usr/bin/env python3
"""Benchmark of the Transformer forward hot path on one MI355X.

Workload (BASELINE.json's metric configuration, "configs[4]"): a 2-layer
pre-LN causal Transformer, B=32 S=100000 D=1024 H=16 (head_dim 64) FFN 4096,
bf16, seeded Xavier-uniform weights (zero biases, LayerNorm 1/0) and N(0,1)
inputs, executed by the plugin model's streamed HIP program as 16 ordered
B=2 chunks.  One "step" is one full B=32 forward; inputs are resident in HBM
before the timed region.

Printed on stdout: ONE JSON line.  ``value`` is the forward latency in ms
(lower is better).  ``roofline`` covers the dominant kernel, the causal
attention: achieved TFLOP/s = algorithmic FLOPs (4*B*H*Dh*S(S+1)/2 per
launch) / the launches' mean duration, timed with HIP events recorded on the
launch stream around every attention call inside the timed region (a call
also runs the key-norm pre-pass, about 1% of it, so the figure is slightly
below the attention kernel's own).
``cpu_baseline`` times the CPU oracle (fp32 official order, query-blocked
attention, as the reference's portable path) on the box's host cores: one
layer of one sequence at the real length S=100000, row-wise work in full and
the attention on query blocks spread over the sequence (every block scores
all keys, so all blocks cost the same); ``value`` scales that measured layer
to the B=32 two-layer forward, an extrapolation labelled as such.
``cpu_configs`` times the CPU oracle on BASELINE's other configurations
(C1, C2 and C4 whole; C3's operators).

``semantic_check`` compares, in the same run, one sequence of the timed
weights through the HIP program with the product's portable program on the
GPU (bf16 and fp32), as the reference does before timing its long-sequence
shape; ``semantic_check.fp32_io`` runs the same weights as an fp32 model
through the mixed program (fp16 projections and HIP attention, HIP mixed
norms) against the fp32 portable program under the official rule, the check
the reference records for its deployed program (ratio 0.2816).  ``resident_gpu`` times C2 and C4 with their registry programs under
the reference's formal protocol (20 warm-up calls, 3 x 100 timed calls).

``roofline.traffic`` is the attention kernel's HBM bytes per launch measured
by rocprofv3 PMC counters (FETCH_SIZE and WRITE_SIZE, each scaled by what
the counter reads for a copy of known size).  Those runs use
``--kernel attention`` and ``--kernel copy`` below; their result is kept in
profiles/attn_fwd_c5_chunk_traffic.md as ``key = value`` lines and is
reported only while ``source_digest`` there equals the digest of the current
attention source and default launch (otherwise null).

``--kernel attention|norm|copy|linear|linear-torch|gelu|gelu-torch|qkv|qkv-torch|boundary|boundary-torch|``
``boundary-ffn|boundary-ffn-torch`` runs one kernel alone at
the workload's per-chunk shape (for rocprofv3 runs) and prints each launch's
duration: attention over a packed [2, S, 3D] QKV view exactly as the model
hands it over, the fused residual+LayerNorm at one chunk's block boundary, a
1 GiB device copy used to calibrate the memory counters, the fused HIP
Linear + bias + exact GELU of the FFN input projection ([2S, D] -> [2S, F]),
the same projection as hipBLASLt F.linear followed by torch's exact GELU, or
the exact GELU alone on the [2S, F] hidden tensor (HIP in place, or torch), or
the packed QKV projection ([2S, D] -> 3 x [2, H, S, 64]): the HIP kernel with
the head-major epilogue and seq-contiguous value, or hipBLASLt F.linear into
the packed [2S, 3D] tensor the default program views, or a residual boundary
with its projection: the fused HIP Linear + residual + LayerNorm kernel, or
hipBLASLt F.linear followed by the HIP residual LayerNorm, for the attention
output projection (D -> D) or the FFN output projection (F -> D).  Attention runs with
the long-sequence program's launch (HIP_LONG_SEQUENCE_ATTENTION_LAUNCH).
``--kernel attention-c4`` runs BASELINE configs[3]'s attention alone (B16 H32
S4096 from the packed QKV view, launch 256/64/8/2) for counter runs.

``config3`` in the JSON line reports BASELINE.json's operator-alone
configuration, timed before the forward on the idle GPU: the attention op
with the long-sequence launch and the residual LayerNorm with its default
launch.
``--kernel attention-c3|norm-c3`` times that configuration alone: causal
attention at B8 H16 S2048 Dh64 under every implemented launch, with V in
[B, H, S, 64] and in seq-contiguous layout, or the fused residual +
LayerNorm on [16384, 1024] under a few launches; each line is the mean of
``--repeat`` back-to-back launches.
``--resident c2|c4`` runs one resident configuration's latency protocol alone
and prints its JSON summary (for a kernel-trace profile of that forward).
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PACKAGE_DIR = ROOT / "ml-guided-program-search-for-shape-specialized-transformer-optimization_amd"
for _path in (PACKAGE_DIR, ROOT):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

METRIC = "fwd latency ms + attn TFLOP/s (% MFMA peak), B=32 S=100k D=1024 H=16 causal"
PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
WORKLOAD = dict(batch=32, seq_len=100_000, d_model=1024, heads=16, ffn_dim=4096, layers=2, microbatch=2)


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


class _Config:
    def __init__(self, batch, seq_len, d_model, heads, ffn_dim, layers):
        self.batch_size = batch
        self.seq_len = seq_len
        self.d_model = d_model
        self.num_heads = heads
        self.ffn_dim = ffn_dim
        self.num_layers = layers
        self.causal = True


def _init_xavier(model, seed: int) -> None:
    """Seeded Xavier-uniform for every projection role (q, k and v separately
    inside the packed qkv_proj), zero biases, LayerNorm weight 1 / bias 0."""

    import torch

    generator = torch.Generator().manual_seed(seed)

    def fill(weight):
        out_features, in_features = weight.shape
        bound = math.sqrt(6.0 / (in_features + out_features))
        return (torch.rand(out_features, in_features, generator=generator) * 2 - 1) * bound

    with torch.no_grad():
        for layer in model.layers:
            d = layer.attention.d_model
            packed = layer.attention.qkv_proj.weight
            for index in range(3):
                packed[index * d : (index + 1) * d].copy_(fill(packed[index * d : (index + 1) * d]))
            for linear in (layer.attention.out_proj, layer.ffn_in, layer.ffn_out):
                linear.weight.copy_(fill(linear.weight))
            for linear in (layer.attention.qkv_proj, layer.attention.out_proj, layer.ffn_in, layer.ffn_out):
                linear.bias.zero_()
        for module in model.modules():
            if isinstance(module, torch.nn.LayerNorm):
                module.weight.fill_(1.0)
                module.bias.zero_()


class _KernelTimer:
    """Wraps a launcher so every call is bracketed by HIP events on the
    current (launch) stream; durations are read after the timed region."""

    def __init__(self, module, name: str):
        self.module = module
        self.name = name
        self.original = getattr(module, name)
        self.events = []
        self.work = []
        self.active = False

    def install(self, work_of):
        import torch

        def wrapped(*args, **kwargs):
            if not self.active:
                return self.original(*args, **kwargs)
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            result = self.original(*args, **kwargs)
            end.record()
            self.events.append((start, end))
            self.work.append(work_of(*args, **kwargs))
            return result

        setattr(self.module, self.name, wrapped)

    def summary(self):
        durations = [start.elapsed_time(end) for start, end in self.events]
        return durations, self.work


def _attention_flops(query, *args, **kwargs) -> float:
    batch, heads, seq, dim = query.shape
    return 4.0 * batch * heads * dim * (seq * (seq + 1) // 2)


def _norm_bytes(value, update, weight, bias, eps, normalized_dtype, *args, **kwargs) -> float:
    import torch

    width = value.shape[-1]
    rows = value.numel() // width
    out_size = torch.empty((), dtype=normalized_dtype).element_size()
    per = 2 * value.element_size() + update.element_size() + out_size
    params = sum(t.numel() * t.element_size() for t in (weight, bias) if t is not None)
    return float(rows * width * per + params)


def gpu_benchmark(steps: int, warmup: int, *, check: bool = True) -> dict:
    import torch

    from solution.kernels.hip import load_library
    from solution.kernels.norm import hip_residual
    from solution.shape14 import hip_streaming_dh64
    from solution.shape14.defaults import hip_streamed_config
    from solution.transformer import UserOptimizedTransformer

    load_library()
    device = torch.device("cuda", 0)
    w = WORKLOAD
    config = _Config(w["batch"], w["seq_len"], w["d_model"], w["heads"], w["ffn_dim"], w["layers"])
    model = UserOptimizedTransformer(config)
    _init_xavier(model, seed=1234)
    model = model.to(device=device, dtype=torch.bfloat16).eval()
    program = hip_streamed_config(microbatch_size=w["microbatch"])
    model.configure_execution(config=program)

    generator = torch.Generator(device=device).manual_seed(1234)
    x = torch.randn(w["batch"], w["seq_len"], w["d_model"], generator=generator, device=device,
                    dtype=torch.bfloat16)
    torch.cuda.synchronize()
    log(f"input resident: {tuple(x.shape)} bf16, program {program.config_id}")

    attention_timer = _KernelTimer(hip_streaming_dh64, "_launch")
    attention_timer.install(_attention_flops)
    norm_timer = _KernelTimer(hip_residual, "_launch_residual")
    norm_timer.install(_norm_bytes)

    with torch.inference_mode():
        # Peak HBM of one B=2 chunk (same program, one microbatch).
        chunk = x[: w["microbatch"]].contiguous()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(device)
        before = torch.cuda.memory_allocated(device)
        model(chunk)
        torch.cuda.synchronize()
        peak_chunk = torch.cuda.max_memory_allocated(device) - before
        del chunk
        log(f"peak HBM above resident tensors for one B=2 chunk: {peak_chunk / 2**30:.2f} GiB")

        for index in range(warmup):
            model(x)
            torch.cuda.synchronize()
            log(f"warmup step {index + 1}/{warmup} done")

        attention_timer.active = True
        norm_timer.active = True
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for index in range(steps):
            output = model(x)
            log(f"timed step {index + 1}/{steps} issued")
        end.record()
        torch.cuda.synchronize()
        attention_timer.active = False
        norm_timer.active = False
        total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / steps
    if not bool(torch.isfinite(output).all()):
        raise RuntimeError("the timed forward produced non-finite values")
    del output
    semantic = semantic_check(model, x) if check else None

    durations, flops = attention_timer.summary()
    attention_ms = sum(durations) / len(durations)
    attention_flops = sum(flops) / len(flops)
    attention_tflops = attention_flops / (attention_ms * 1e-3) / 1e12
    norm_durations, norm_work = norm_timer.summary()
    norm_us = 1e3 * sum(norm_durations) / len(norm_durations)
    norm_gbs = (sum(norm_work) / len(norm_work)) / (norm_us * 1e-6) / 1e9

    layers, batch, seq, width, ffn = w["layers"], w["batch"], w["seq_len"], w["d_model"], w["ffn_dim"]
    model_flops = layers * (2 * batch * seq * seq * width + 8 * batch * seq * width**2 + 4 * batch * seq * width * ffn)
    log(f"{ms_per_step:.1f} ms/step; attention {attention_ms:.3f} ms/launch {attention_tflops:.1f} TFLOP/s; "
        f"norm {norm_us:.1f} us/launch {norm_gbs:.0f} GB/s")
    return {
        "ms_per_step": ms_per_step,
        "attention_ms_per_launch": attention_ms,
        "attention_launches_per_step": len(durations) // steps,
        "attention_flops_per_launch": attention_flops,
        "attention_tflops": attention_tflops,
        "attention_share_of_step": sum(durations) / total_ms,
        "norm_us_per_launch": norm_us,
        "norm_bytes_per_launch": sum(norm_work) / len(norm_work),
        "norm_gbs": norm_gbs,
        "peak_hbm_bytes_per_chunk": int(peak_chunk),
        "model_flops": model_flops,
        "config_id": program.config_id,
        "semantic_check": semantic,
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "attn_fwd_c5_chunk_traffic.md"
ATTENTION_SOURCES = tuple(
    PACKAGE_DIR / "csrc" / name for name in ("attention_kernel.hpp", "attention_fwd.hip", "attention_scaled.hip")
)


def attention_source_digest() -> str:
    """Digest of what the traffic figure depends on: the attention kernel
    sources and the launch the long-sequence program uses."""

    from solution.config import HIP_LONG_SEQUENCE_ATTENTION_LAUNCH

    digest = hashlib.sha256()
    for path in ATTENTION_SOURCES:
        digest.update(path.read_bytes())
    digest.update(repr(HIP_LONG_SEQUENCE_ATTENTION_LAUNCH).encode())
    return digest.hexdigest()[:16]


def measured_traffic() -> float | None:
    """HBM bytes per attention launch from the committed PMC summary, or None
    when it is absent or was measured on other kernel source."""

    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None
    fields = dict(re.findall(r"^(\w+) = (\S+)\s*$", text, flags=re.MULTILINE))
    if fields.get("source_digest") != attention_source_digest():
        log("traffic profile is for other attention source; roofline.traffic = null")
        return None
    try:
        return float(fields["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def _config3_cases(kind: str, device, *, launches=None, abi: bool = False):
    """BASELINE configs[2], the operators alone: causal attention at B8 H16
    S2048 Dh64 (Q, K, V N(0,1)/sqrt(64), scale 1/8; V both [B, H, S, 64]
    contiguous, which the kernel reads as given, and seq-contiguous, which
    the op first copies key-major into its workspace), or the fused
    residual + LayerNorm on [16384, 1024] bf16 N(0,1) over rotating buffers.
    Returns (label, run, work) triples: FLOPs or bytes per launch.

    ``abi``: each launch calls the C-ABI entry point (the drop-in boundary)
    on preallocated outputs and workspace, so back-to-back launches measure
    the device-side rate; otherwise the Python operator, which allocates its
    outputs per call (at ~25 us per norm launch its host time can leave the
    GPU idle between launches)."""

    import torch

    from solution.kernels.hip._library import check_status, dtype_code, load_library, stream_handle
    from solution.kernels.norm import hip_residual
    from solution.shape14 import hip_streaming_dh64

    library = load_library()
    stream = stream_handle(device)
    generator = torch.Generator(device=device).manual_seed(1234)
    cases = []
    if kind == "attention-c3":
        q, k, v = (
            (torch.randn(8, 16, 2048, 64, generator=generator, device=device) / 8).to(torch.bfloat16)
            for _ in range(3)
        )
        flops = _attention_flops(q)
        # the same V stored seq-contiguous ([B, H, 64, S] transposed view), as
        # the native QKV projection's seq-major option hands it over
        v_seq_major = v.transpose(-1, -2).contiguous().transpose(-1, -2)
        output = torch.empty(8, 2048, 16 * 64, device=device, dtype=torch.bfloat16)
        code = dtype_code(torch.bfloat16)
        if launches is None:
            launches = [
                (block_m, warps, stages)
                for block_m in (128, 256, 512)
                for warps in (4, 8)
                for stages in (1, 2, 3)
                if hip_streaming_dh64.launch_config_is_valid(block_m, 64, warps, stages)
            ]

        def abi_launch(value, block_m, warps, stages, workspace):
            status = library.sah_causal_attention_bsd(
                q.data_ptr(), k.data_ptr(), value.data_ptr(), output.data_ptr(), 8, 16, 2048, 64,
                *q.stride()[:3], *k.stride()[:3], *value.stride(), output.stride(0), output.stride(1),
                0.125, code, block_m, 64, warps, stages,
                None if workspace is None else workspace.data_ptr(),
                0 if workspace is None else workspace.numel(), stream)
            check_status(status, "sah_causal_attention_bsd")

        for block_m, warps, stages in launches:
            for layout, value in (("V bhsd", v), ("V seq-major", v_seq_major)):
                if abi:
                    need = library.sah_causal_attention_workspace_bytes(
                        8, 16, 2048, 64, value.stride(2), value.stride(3), code)
                    workspace = torch.empty(need, dtype=torch.uint8, device=device) if need else None
                    run = (lambda bm=block_m, w=warps, st=stages, value=value, ws=workspace:
                           abi_launch(value, bm, w, st, ws))
                else:
                    run = (lambda bm=block_m, w=warps, st=stages, value=value:
                           hip_streaming_dh64.hip_streaming_dh64_causal_attention_bsd(
                               q, k, value, scale=0.125, block_m=bm, block_n=64, num_warps=w, num_stages=st))
                cases.append((f"launch ({block_m}, 64, {warps}, {stages}) {layout}", run, flops))
    else:
        # 6 input pairs and 6 output pairs: every launch touches buffers last
        # used ~0.8 GB earlier, more than twice the 256 MB Infinity Cache, so
        # the rate is HBM's, not MALL's
        sets = 6
        inputs = [
            (torch.randn(16384, 1024, generator=generator, device=device, dtype=torch.bfloat16),
             torch.randn(16384, 1024, generator=generator, device=device, dtype=torch.bfloat16))
            for _ in range(sets)
        ]
        outputs = [(torch.empty(16384, 1024, device=device, dtype=torch.bfloat16),
                    torch.empty(16384, 1024, device=device, dtype=torch.bfloat16)) for _ in range(sets)]
        counter = [0]
        layer_norm = torch.nn.LayerNorm(1024).to(device=device, dtype=torch.bfloat16)
        nbytes = _norm_bytes(*inputs[0], layer_norm.weight, layer_norm.bias, 1e-5, torch.bfloat16)
        code = dtype_code(torch.bfloat16)

        def rotating(block_rows, warps):
            index = counter[0] % sets
            counter[0] += 1
            (value, update), (residual, normalized) = inputs[index], outputs[index]
            if abi:
                status = library.sah_residual_norm(
                    value.data_ptr(), update.data_ptr(), layer_norm.weight.data_ptr(), layer_norm.bias.data_ptr(),
                    residual.data_ptr(), normalized.data_ptr(), 16384, 1024, 1e-5, code, code, code, code,
                    0, block_rows, warps, stream)
                check_status(status, "sah_residual_norm")
            else:
                hip_residual.hip_residual_layer_norm(
                    value, update, layer_norm, block_rows=block_rows, num_warps=warps, out=normalized)

        for block_rows, warps in launches or ((2, 2), (4, 4), (8, 8), (16, 8)):
            cases.append((
                f"launch ({block_rows} rows, {warps} waves)",
                lambda br=block_rows, w=warps: rotating(br, w),
                nbytes,
            ))
    return cases


def _back_to_back_ms(run, repeat: int, *, warmup: int = 1, trials: int = 1) -> float:
    """Mean HIP-event time per launch of `repeat` back-to-back launches (the
    host enqueues faster than the GPU drains, so host-side call overhead is
    hidden) after `warmup` untimed launches; the median over `trials`."""

    import torch

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    means = []
    for _ in range(trials):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(repeat):
            run()
        end.record()
        torch.cuda.synchronize()
        means.append(start.elapsed_time(end) / repeat)
    return sorted(means)[len(means) // 2]


def config3_alone(kind: str, repeat: int, launches=None) -> int:
    """Time every implemented launch of one operator-alone case through the
    C ABI and through the Python operator; print each mean launch time and
    its rate."""

    import torch

    from solution.kernels.hip import load_library

    load_library()
    with torch.inference_mode():
        device = torch.device("cuda", 0)
        for abi in (True, False):
            how = "C-ABI launches" if abi else "Python operator"
            for label, run, work in _config3_cases(kind, device, abi=abi, launches=launches):
                ms = _back_to_back_ms(run, repeat)
                if kind == "attention-c3":
                    rate = f"{work / ms / 1e9:.1f} TFLOP/s ({100 * work / ms / 1e9 / PEAK_BF16_TFLOPS:.1f}% of peak)"
                else:
                    rate = f"{work / ms / 1e6:.1f} GB/s ({100 * work / ms / 1e6 / PEAK_HBM_GBS:.1f}% of 8 TB/s)"
                print(f"{kind} {label}: {ms:.4f} ms per launch (mean of {repeat} back-to-back, {how}), {rate}",
                      flush=True)
    return 0


def config3_summary(repeat: int = 100, warmup: int = 2000, trials: int = 5) -> dict:
    """The operator-alone figures reported beside the forward: attention with
    the long-sequence launch (V in the reference's [B, H, S, 64] layout, read
    as given, and a seq-contiguous V^T, its key-major copy included), the
    norm with its default launch.
    Each figure is the median of `trials` means of `repeat` back-to-back
    launches.  The first case runs `warmup` untimed launches (about 0.2 s)
    that bring the idle chip to its clock: the first hundreds of launches
    measured up to 15% slower."""

    import torch

    from solution.config import HIP_LONG_SEQUENCE_ATTENTION_LAUNCH as L
    from solution.kernels.norm.hip_residual import DEFAULT_BLOCK_ROWS, DEFAULT_NUM_WARPS

    device = torch.device("cuda", 0)
    with torch.inference_mode():
        launch = [(L.block_m, L.num_warps, L.num_stages)]
        norm_launch = [(DEFAULT_BLOCK_ROWS, DEFAULT_NUM_WARPS)]
        (_, run_bhsd, flops), (_, run_seq, _) = _config3_cases("attention-c3", device, launches=launch, abi=True)
        attention_ms = _back_to_back_ms(run_bhsd, repeat, warmup=warmup, trials=trials)
        attention_seq_ms = _back_to_back_ms(run_seq, repeat, warmup=repeat, trials=trials)
        (_, run_op, _), _ = _config3_cases("attention-c3", device, launches=launch)
        op_attention_ms = _back_to_back_ms(run_op, repeat, warmup=repeat, trials=trials)
        del run_bhsd, run_seq, run_op
        ((_, run_norm, nbytes),) = _config3_cases("norm-c3", device, launches=norm_launch, abi=True)
        norm_ms = _back_to_back_ms(run_norm, repeat, warmup=repeat, trials=trials)
        ((_, run_norm_op, _),) = _config3_cases("norm-c3", device, launches=norm_launch)
        op_norm_ms = _back_to_back_ms(run_norm_op, repeat, warmup=repeat, trials=trials)
    tflops = flops / attention_ms / 1e9
    tflops_seq = flops / attention_seq_ms / 1e9
    gbs = nbytes / norm_ms / 1e6
    log(f"config 3: attention {1e3 * attention_ms:.1f} us ({1e3 * attention_seq_ms:.1f} us seq-contiguous V), "
        f"norm {1e3 * norm_ms:.1f} us through the C ABI; Python operators {1e3 * op_attention_ms:.1f} us, "
        f"{1e3 * op_norm_ms:.1f} us")
    return {
        "workload": "operators alone (BASELINE configs[2]): attention B8 H16 S2048 Dh64, norm [16384, 1024]",
        "timing": f"median of {trials} means of {repeat} back-to-back C-ABI launches on preallocated outputs "
                  f"(the drop-in boundary), HIP events, after {warmup} warm-up attention launches, before the "
                  f"forward; python_operator_* the same launches through the Python operators, which allocate "
                  f"their outputs per call",
        "python_operator_attention_us": round(1e3 * op_attention_ms, 2),
        "python_operator_norm_us": round(1e3 * op_norm_ms, 2),
        "attention_launch": [L.block_m, L.block_n, L.num_warps, L.num_stages],
        "attention_us": round(1e3 * attention_ms, 2),
        "attention_tflops": round(tflops, 1),
        "attention_pct_mfma_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "attention_seq_contiguous_v_us": round(1e3 * attention_seq_ms, 2),
        "attention_seq_contiguous_v_pct_mfma_peak": round(100 * tflops_seq / PEAK_BF16_TFLOPS, 2),
        "norm_us": round(1e3 * norm_ms, 2),
        "norm_gbs": round(gbs, 1),
        "norm_pct_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
    }


def kernel_alone(kind: str, repeat: int, data: str = "random") -> int:
    """Run one kernel alone at the workload's per-chunk shape; print the
    HIP-event duration of every launch.  ``data="constant"`` fills the
    attention's packed QKV with one value instead of N(0,1) (same
    instructions, far fewer switching bits: the chip's power-limited clock
    then rises, which the clock counters of a profile show)."""

    import torch

    from solution.config import HIP_LONG_SEQUENCE_ATTENTION_LAUNCH
    from solution.kernels.hip import load_library
    from solution.kernels.norm import hip_residual
    from solution.shape14 import hip_streaming_dh64

    load_library()
    device = torch.device("cuda", 0)
    w = WORKLOAD
    batch, seq, width, heads = w["microbatch"], w["seq_len"], w["d_model"], w["heads"]
    generator = torch.Generator(device=device).manual_seed(7)
    with torch.inference_mode():
        if kind == "attention":
            packed = torch.randn(batch, seq, 3 * width, generator=generator, device=device,
                                 dtype=torch.bfloat16)
            if data == "constant":
                packed.fill_(0.25)
            q, k, v = (t.transpose(1, 2) for t in packed.unflatten(-1, (3, heads, width // heads)).unbind(dim=2))
            scale = 1.0 / math.sqrt(width // heads)
            launch = HIP_LONG_SEQUENCE_ATTENTION_LAUNCH
            run = lambda: hip_streaming_dh64.hip_streaming_dh64_causal_attention_bsd(
                q, k, v, scale=scale, block_m=launch.block_m, block_n=launch.block_n,
                num_warps=launch.num_warps, num_stages=launch.num_stages)
            work = f"{_attention_flops(q) / 1e12:.3f} TFLOP per launch"
        elif kind == "attention-c4":
            # BASELINE configs[3]'s attention, B16 H32 S4096, from the packed
            # QKV view the resident program hands over, with its registry
            # launch (256/64/8/2, preparation and scaled-key path).
            c4_batch, c4_seq, c4_width, c4_heads = RESIDENT_SHAPES["c4"][:4]
            packed = torch.randn(c4_batch, c4_seq, 3 * c4_width, generator=generator, device=device,
                                 dtype=torch.bfloat16)
            q, k, v = (t.transpose(1, 2) for t in packed.unflatten(-1, (3, c4_heads, c4_width // c4_heads)).unbind(dim=2))
            scale = 1.0 / math.sqrt(c4_width // c4_heads)
            run = lambda: hip_streaming_dh64.hip_streaming_dh64_causal_attention_bsd(
                q, k, v, scale=scale, block_m=256, block_n=64, num_warps=8, num_stages=2)
            work = f"{_attention_flops(q) / 1e12:.3f} TFLOP per launch"
        elif kind == "norm":
            value = torch.randn(batch * seq, width, generator=generator, device=device, dtype=torch.bfloat16)
            update = torch.randn_like(value)
            layer_norm = torch.nn.LayerNorm(width).to(device=device, dtype=torch.bfloat16)
            run = lambda: hip_residual.hip_residual_layer_norm(value, update, layer_norm)
            work = f"{_norm_bytes(value, update, layer_norm.weight, layer_norm.bias, 1e-5, torch.bfloat16) / 1e9:.4f} GB per launch"
        elif kind == "copy":
            source = torch.randn(2**29, generator=generator, device=device, dtype=torch.bfloat16)
            target = torch.empty_like(source)
            run = lambda: target.copy_(source)
            work = "1 GiB read + 1 GiB written per launch"
        elif kind in ("linear", "linear-torch"):
            from solution.kernels.ffn import prevalidated_hip_linear_exact_gelu

            rows, ffn = batch * seq, w["ffn_dim"]
            x = torch.randn(rows, width, generator=generator, device=device, dtype=torch.bfloat16)
            bound = math.sqrt(6.0 / (width + ffn))
            weight = ((torch.rand(ffn, width, generator=generator, device=device) * 2 - 1) * bound).to(torch.bfloat16)
            bias = torch.zeros(ffn, device=device, dtype=torch.bfloat16)
            if kind == "linear":
                run = lambda: prevalidated_hip_linear_exact_gelu(x, weight, bias)
            else:
                run = lambda: torch.nn.functional.gelu(torch.nn.functional.linear(x, weight, bias), approximate="none")
            work = f"{2 * rows * width * ffn / 1e12:.3f} TFLOP per launch"
        elif kind in ("qkv", "qkv-torch"):
            from solution.kernels.projection import prevalidated_hip_qkv_native_bhsd

            x = torch.randn(batch, seq, width, generator=generator, device=device, dtype=torch.bfloat16)
            bound = math.sqrt(6.0 / (4 * width))
            weight = ((torch.rand(3 * width, width, generator=generator, device=device) * 2 - 1) * bound).to(torch.bfloat16)
            bias = torch.zeros(3 * width, device=device, dtype=torch.bfloat16)
            if kind == "qkv":
                run = lambda: prevalidated_hip_qkv_native_bhsd(x, weight, bias, num_heads=heads, value_layout="seq_major")
            else:
                run = lambda: torch.nn.functional.linear(x, weight, bias)
            work = f"{2 * batch * seq * width * 3 * width / 1e12:.3f} TFLOP per launch"
        elif kind.startswith("boundary"):
            from solution.kernels.boundary import block_rows_for, hip_linear_residual_norm

            in_features = w["ffn_dim"] if kind.startswith("boundary-ffn") else width
            x = torch.randn(batch, seq, in_features, generator=generator, device=device, dtype=torch.bfloat16)
            bound = math.sqrt(6.0 / (width + in_features))
            weight = ((torch.rand(width, in_features, generator=generator, device=device) * 2 - 1) * bound).to(torch.bfloat16)
            bias = torch.zeros(width, device=device, dtype=torch.bfloat16)
            value = torch.randn(batch, seq, width, generator=generator, device=device, dtype=torch.bfloat16)
            layer_norm = torch.nn.LayerNorm(width).to(device=device, dtype=torch.bfloat16)
            if kind.endswith("-torch"):
                run = lambda: hip_residual.hip_residual_layer_norm(
                    value, torch.nn.functional.linear(x, weight, bias), layer_norm)
            else:
                run = lambda: hip_linear_residual_norm(
                    x, weight, bias, value, layer_norm, block_rows=block_rows_for(width), num_warps=8)
            work = f"{2 * batch * seq * in_features * width / 1e12:.3f} TFLOP + {8 * batch * seq * width / 1e9:.3f} GB per launch"
        elif kind in ("gelu", "gelu-torch"):
            from solution.kernels.ffn import prevalidated_hip_exact_gelu

            hidden = torch.randn(batch * seq, w["ffn_dim"], generator=generator, device=device,
                                 dtype=torch.bfloat16)
            if kind == "gelu":
                run = lambda: prevalidated_hip_exact_gelu(hidden, out=hidden)
            else:
                run = lambda: torch.nn.functional.gelu(hidden, approximate="none")
            work = f"{2 * 2 * hidden.numel() / 1e9:.3f} GB per launch"
        else:
            raise SystemExit(f"unknown kernel {kind!r}")
        torch.cuda.synchronize()
        for index in range(repeat):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            run()
            end.record()
            torch.cuda.synchronize()
            print(f"{kind} launch {index + 1}/{repeat}: {start.elapsed_time(end):.3f} ms ({work})", flush=True)
    return 0


def _cpu_cores() -> tuple[int, int, float | None]:
    """(threads used, CPUs in this process's affinity set, cgroup CPU quota):
    every CPU of the affinity set, unless the cgroup's quota allows fewer."""

    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        limit, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if limit != "max":
            quota = int(limit) / int(period)
    except (OSError, ValueError):
        quota = None
    threads = affinity if quota is None else max(1, min(affinity, math.floor(quota)))
    return threads, affinity, quota


def _cpu_samples(run, *, warmup: int, samples: int) -> list[float]:
    """Wall-clock seconds of `samples` calls after `warmup` untimed ones, with
    time.perf_counter_ns (the official CPU method,
    official/torch_transformer_benchmark.py:501-506)."""

    for _ in range(warmup):
        run()
    times = []
    for _ in range(samples):
        start = time.perf_counter_ns()
        run()
        times.append((time.perf_counter_ns() - start) / 1e9)
    return times


def _median(values):
    ordered = sorted(values)
    middle = len(ordered) // 2
    return ordered[middle] if len(ordered) % 2 else 0.5 * (ordered[middle - 1] + ordered[middle])


def cpu_long_sequence(threads: int, *, blocks_timed: int = 96, full_layer: bool = False) -> dict:
    """The CPU oracle on one layer of one sequence at the real length
    S = 100000 (fp32, official op order, the reference portable path's
    query-blocked attention: every 128-row block scores all S keys, so every
    block does the same work wherever it sits).

    Measured: the row-wise work of the layer in full (norm1 and the q, k, v
    projections over all S rows; out projection, residual, norm2 and FFN over
    all S rows), the final LayerNorm, and ``blocks_timed`` query blocks spread
    evenly over the sequence; the layer's attention is their mean times the
    number of blocks.  With ``full_layer`` the whole layer's attention is run
    instead (about two minutes).  The full B=32 forward is 32 sequences x
    (2 layers + final norm): an extrapolation of the measured layer, labelled
    as such."""

    import torch

    from oracle.forward import (
        TransformerConfig,
        attention_inputs,
        final_norm,
        generate_input,
        layer_output,
        query_block_rows,
        xavier_init_weights,
    )

    torch.set_num_threads(threads)
    w = WORKLOAD
    seq, heads, block = w["seq_len"], w["heads"], 128
    config = TransformerConfig(1, seq, w["d_model"], heads, w["ffn_dim"], 1, True)
    state = xavier_init_weights(config, seed=1234)
    x = generate_input(config, seed=1234)
    scale = (w["d_model"] // heads) ** -0.5
    starts = list(range(0, seq, block))
    if full_layer:
        chosen = starts
    else:
        chosen = [starts[(i * (len(starts) - 1)) // (blocks_timed - 1)] for i in range(blocks_timed)]
    with torch.inference_mode():
        small = TransformerConfig(1, 256, w["d_model"], heads, w["ffn_dim"], 1, True)
        q, k, v = attention_inputs(state, x[:, :256], 0, heads)  # warm the code paths
        layer_output(state, x[:, :256], query_block_rows(q, k, v, scale, 0, 256), 0)
        del small
        t0 = time.perf_counter_ns()
        q, k, v = attention_inputs(state, x, 0, heads)
        t_inputs = (time.perf_counter_ns() - t0) / 1e9
        context = torch.zeros_like(q)
        # one untimed block at the real size: its first call pays the
        # allocation of the [H, 128, S] temporaries
        query_block_rows(q, k, v, scale, chosen[-1], min(chosen[-1] + block, seq))
        block_times = []
        for start in chosen:
            stop = min(start + block, seq)
            t0 = time.perf_counter_ns()
            context[..., start:stop, :] = query_block_rows(q, k, v, scale, start, stop)
            block_times.append((time.perf_counter_ns() - t0) / 1e9)
        t0 = time.perf_counter_ns()
        out = layer_output(state, x, context, 0)
        t_output = (time.perf_counter_ns() - t0) / 1e9
        t0 = time.perf_counter_ns()
        final_norm(state, out)
        t_final = (time.perf_counter_ns() - t0) / 1e9
    log(f"cpu layer: block times {', '.join(f'{1e3 * t:.0f}' for t in block_times[:8])} ... ms")
    attention_s = sum(block_times) if full_layer else len(starts) * sum(block_times) / len(block_times)
    layer_s = t_inputs + attention_s + t_output
    forward_s = w["batch"] * (w["layers"] * layer_s + t_final)
    how = ("every query block" if full_layer else
           f"{len(chosen)} of its {len(starts)} query blocks (each scores all {seq} keys: equal work), "
           f"mean {1e3 * sum(block_times) / len(block_times):.1f} ms per block")
    return {
        "layer_ms": round(1e3 * layer_s, 1),
        "layer_is_measured": full_layer,
        "attention_blocks_timed": len(chosen),
        "attention_blocks": len(starts),
        "forward_ms": round(1e3 * forward_s, 1),
        "sample": (
            f"fp32 CPU oracle (official op order, query-blocked attention), one layer of one sequence at "
            f"S={seq} D{w['d_model']} H{heads} F{w['ffn_dim']}, measured: row-wise work in full "
            f"({1e3 * (t_inputs + t_output):.0f} ms), attention over {how}, layer {1e3 * layer_s:.0f} ms; "
            f"the B={w['batch']} forward is an extrapolation: {w['batch']} sequences x ({w['layers']} layers "
            f"+ final norm {1e3 * t_final:.0f} ms)"
        ),
    }


def cpu_configs(threads: int) -> dict:
    """The CPU oracle (fp32) on BASELINE's other configurations: C1, C2 and C4
    whole forwards and C3's operators (on inputs widened from the bf16 ones
    the GPU figures use).  Warm-up and median per the official CPU method
    where a sample takes seconds; C4 (about 20 s) is one sample."""

    import torch

    from oracle.forward import (
        TransformerConfig,
        default_init_weights,
        forward,
        generate_input,
        query_block_causal_attention,
        xavier_init_weights,
    )
    torch.set_num_threads(threads)
    out = {}
    with torch.inference_mode():
        c1 = TransformerConfig(2, 128, 256, 4, 1024, 2, True)
        state, x = default_init_weights(c1, seed=1234), generate_input(c1, seed=1234)
        times = _cpu_samples(lambda: forward(state, x, c1), warmup=2, samples=5)
        out["c1"] = {"ms": round(1e3 * _median(times), 3), "what": "whole forward B2 S128 D256 H4 F1024 L2",
                     "samples": 5}
        c2 = TransformerConfig(64, 256, 512, 8, 2048, 4, True)
        state, x = xavier_init_weights(c2, seed=1234), generate_input(c2, seed=1234)
        times = _cpu_samples(lambda: forward(state, x, c2), warmup=1, samples=3)
        out["c2"] = {"ms": round(1e3 * _median(times), 1), "what": "whole forward B64 S256 D512 H8 F2048 L4",
                     "samples": 3}
        generator = torch.Generator().manual_seed(1234)
        q, k, v = ((torch.randn(8, 16, 2048, 64, generator=generator) / 8).to(torch.bfloat16).float()
                   for _ in range(3))
        times = _cpu_samples(lambda: query_block_causal_attention(q, k, v, 0.125), warmup=1, samples=5)
        value = torch.randn(16384, 1024, generator=generator).to(torch.bfloat16).float()
        update = torch.randn(16384, 1024, generator=generator).to(torch.bfloat16).float()
        gamma, beta = torch.ones(1024), torch.zeros(1024)

        def boundary():  # the reference's torch boundary: add, then LayerNorm
            residual = value + update
            return residual, torch.nn.functional.layer_norm(residual, (1024,), gamma, beta, 1e-5)

        norm_times = _cpu_samples(boundary, warmup=1, samples=5)
        out["c3"] = {"attention_ms": round(1e3 * _median(times), 2), "norm_ms": round(1e3 * _median(norm_times), 2),
                     "what": "attention B8 H16 S2048 Dh64 (query-blocked order) and residual add + LayerNorm "
                             "[16384, 1024], fp32",
                     "samples": 5}
        # C4 in full (about 20 s on 16 host threads), one sample
        c4 = TransformerConfig(16, 4096, 2048, 32, 8192, 2, True)
        state, x = xavier_init_weights(c4, seed=1234), generate_input(c4, seed=1234)
        times = _cpu_samples(lambda: forward(state, x, c4, attention="query_block"), warmup=0, samples=1)
        out["c4"] = {"ms": round(1e3 * times[0], 1),
                     "what": "whole forward B16 S4096 D2048 H32 F8192 L2 (query-blocked order)", "samples": 1}
    return out


def _deployed_program(d_model: int, seq_len: int):
    """The committed registry's program for the BASELINE shape of this width
    and length."""

    from deployment.registry import DEFAULT_DEPLOYED_CONFIGS_PATH
    from solution.config import ConfigSpec

    document = json.loads(DEFAULT_DEPLOYED_CONFIGS_PATH.read_text(encoding="utf-8"))
    for bundle in document["bundles"]:
        for entry in bundle["entries"]:
            shape = entry["shape"]
            if shape["qkv_dim"] == d_model and shape["seq_len"] == seq_len and shape["dtype"] == "bfloat16":
                return ConfigSpec.from_dict(entry["config"])
    raise RuntimeError(f"no registry entry for D={d_model} S={seq_len}")


def _percentile(values, q):
    ordered = sorted(values)
    position = (len(ordered) - 1) * q
    lower, upper = math.floor(position), math.ceil(position)
    return ordered[lower] + (ordered[upper] - ordered[lower]) * (position - lower)


# The headline's resident configurations C2 and C4 as (B, S, D, H, F, L), bf16.
RESIDENT_SHAPES = {"c2": (64, 256, 512, 8, 2048, 4), "c4": (16, 4096, 2048, 32, 8192, 2)}


def _latency_rounds(model, x, *, warmup: int, repeats: int, rounds: int):
    """The reference's latency protocol on one model: ``warmup`` calls, then
    ``rounds`` rounds of ``repeats`` calls with HIP events around every call
    and one synchronization per round.  Returns the per-call GPU intervals
    (ms) and the host time each call took to return (ms, no synchronization:
    the time the host spends submitting the forward's launches)."""

    import time

    import torch

    samples, host = [], []
    for _ in range(warmup):
        model(x)
    torch.cuda.synchronize()
    for _ in range(rounds):
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
        for index in range(repeats):
            starts[index].record()
            t0 = time.perf_counter()
            model(x)
            host.append((time.perf_counter() - t0) * 1e3)
            ends[index].record()
        torch.cuda.synchronize()
        samples.extend(a.elapsed_time(b) for a, b in zip(starts, ends))
    return samples, host


def _latency_summary(samples: list, repeats: int) -> dict:
    median = _median(samples)
    slow = [i for i, t in enumerate(samples) if t > 1.1 * median]
    return {
        "median_ms": round(median, 4),
        "p90_ms": round(_percentile(samples, 0.9), 4),
        "mean_ms": round(sum(samples) / len(samples), 4),
        "min_ms": round(min(samples), 4),
        "max_ms": round(max(samples), 4),
        "calls_over_1.1x_median": len(slow),
        "of_them_in_first_10_of_a_round": sum(1 for i in slow if i % repeats < 10),
    }


def resident_latency(shape: tuple, *, warmup: int = 20, repeats: int = 100, rounds: int = 3,
                     graph: bool = False) -> dict:
    """GPU forward latency of a resident configuration under the reference's
    formal protocol (benchmarking/protocols.py:116-117: 20 warm-up calls,
    then 3 rounds of 100; official/torch_transformer_benchmark.py:477-506:
    events recorded around every call of a round, one synchronization per
    round), with the registry's program for the shape, bf16, seeded
    Xavier-uniform weights and N(0,1) input.

    Beside the GPU intervals it reports the host time per call (how long
    ``model(x)`` takes to return: the submission of the forward's launches)
    and where the slow calls fall.  An interval reads above the kernels' own
    time when the host submits more slowly than the GPU runs, so a host
    close to the GPU's rate shows its jitter in the tail.  ``graph``: the
    same protocol once more with the program's runtime set to HIP-graph
    replay (one launch per forward), which takes the host out of the
    interval."""

    import dataclasses

    import torch

    from solution.config import RuntimeBackend
    from solution.transformer import UserOptimizedTransformer

    batch, seq, width, heads, ffn, layers = shape
    device = torch.device("cuda", 0)
    model = UserOptimizedTransformer(_Config(batch, seq, width, heads, ffn, layers))
    _init_xavier(model, seed=1234)
    model = model.to(device=device, dtype=torch.bfloat16).eval()
    program = _deployed_program(width, seq)
    model.configure_execution(config=program)
    generator = torch.Generator(device=device).manual_seed(1234)
    x = torch.randn(batch, seq, width, generator=generator, device=device, dtype=torch.bfloat16)
    with torch.inference_mode():
        samples, host = _latency_rounds(model, x, warmup=warmup, repeats=repeats, rounds=rounds)
        graph_summary = None
        if graph and program.schedule.runtime is not RuntimeBackend.CUDA_GRAPH:
            replayed = dataclasses.replace(
                program, schedule=dataclasses.replace(program.schedule, runtime=RuntimeBackend.CUDA_GRAPH))
            model.configure_execution(config=replayed)
            graph_samples, graph_host = _latency_rounds(model, x, warmup=warmup, repeats=repeats, rounds=rounds)
            graph_summary = {
                "program": replayed.config_id,
                **_latency_summary(graph_samples, repeats),
                "host_median_ms": round(_median(graph_host), 4),
            }
    del model, x
    result = {
        "workload": f"B{batch} S{seq} D{width} H{heads} F{ffn} L{layers} bf16",
        "program": program.config_id,
        **_latency_summary(samples, repeats),
        "host_median_ms": round(_median(host), 4),
        "host_p90_ms": round(_percentile(host, 0.9), 4),
        "samples": len(samples),
        "protocol": f"{warmup} warm-up calls, {rounds} rounds x {repeats} calls, HIP events per call",
    }
    if graph_summary is not None:
        result["graph_replay"] = graph_summary
    return result


def semantic_check(model, x) -> dict:
    """The measured program's output checked in the same run, as the
    reference does before it times its long-sequence shape
    (benchmarking/shape14_measure.py:139-162): one sequence (B=1) at the full
    length through the program's inner (one-sequence) schedule, against the
    product's portable reference-order program (query-blocked torch
    attention, torch norms) run on the GPU in bf16 and in fp32 from the same
    weights.  ``passed`` is the model-level rule of autotune.accuracy (no less
    accurate than the bf16 reference path against fp32); the elementwise gates
    and the reference's continuous ratio (<= 1 passes) are reported beside
    it."""

    import torch

    from autotune.accuracy import gate_ratio, summarize_errors, summary_no_less_accurate
    from solution.config import portable_streamed_config
    from solution.shape14.defaults import hip_deployed_shape14_config, hip_mixed_streamed_config, hip_streamed_config
    from solution.transformer import UserOptimizedTransformer

    device = x.device
    state = model.state_dict()
    sample = x[:1].contiguous()

    def run(program, dtype):
        other = UserOptimizedTransformer(model.config)
        other.load_state_dict(state)
        other = other.to(device=device, dtype=dtype).eval()
        other.configure_execution(config=program)
        with torch.inference_mode():
            out = other(sample.to(dtype))
        torch.cuda.synchronize()
        del other
        return out.float()

    candidate = run(hip_streamed_config(microbatch_size=1), torch.bfloat16)
    reference_path = run(portable_streamed_config(), torch.bfloat16)
    exact = run(portable_streamed_config(), torch.float32)
    # fp32 I/O with fp16 internals: the reference's own check of its deployed
    # long-sequence program (fp32 model, fp16 projections and attention)
    # against the fp32 portable program, here with the HIP kernels: that
    # program's shape (fp32 FFN output projection and norms), and the one with
    # fp16 branches throughout (HIP mixed norms).
    fp32_io = {}
    for name, factory in (("deployed_shape14", hip_deployed_shape14_config), ("mixed", hip_mixed_streamed_config)):
        output = run(factory(microbatch_size=1), torch.float32)
        ratio = gate_ratio(output, exact, atol=0.002, rtol=0.02)
        errors = summarize_errors(output, exact, atol=0.002, rtol=0.02)
        fp32_io[name] = {"program": factory.__name__, "official_ratio_rtol0.02_atol0.002": round(ratio, 4),
                         "official_passed": bool(ratio <= 1.0), "max_abs": round(errors.max_abs, 6),
                         "mean_abs": round(errors.mean_abs, 7)}
        del output
    # The same check on the reference's own Shape 14 (F=1024, PyTorch default
    # init, fp32 input): the configuration its recorded ratio was measured on.
    w = WORKLOAD
    shape14_config = _Config(1, w["seq_len"], w["d_model"], w["heads"], 1024, w["layers"])
    torch.manual_seed(1234)
    shape14 = UserOptimizedTransformer(shape14_config)  # PyTorch default init
    shape14_state = shape14.state_dict()
    del shape14
    generator = torch.Generator(device=device).manual_seed(1234)
    shape14_x = torch.randn(1, w["seq_len"], w["d_model"], generator=generator, device=device)
    outputs = []
    for program in (hip_deployed_shape14_config(microbatch_size=1), portable_streamed_config()):
        other = UserOptimizedTransformer(shape14_config)
        other.load_state_dict(shape14_state)
        other = other.to(device=device).eval()
        other.configure_execution(config=program)
        with torch.inference_mode():
            outputs.append(other(shape14_x))
        torch.cuda.synchronize()
        del other
    ratio = gate_ratio(outputs[0], outputs[1], atol=0.002, rtol=0.02)
    errors = summarize_errors(outputs[0], outputs[1], atol=0.002, rtol=0.02)
    fp32_io["reference_shape14"] = {
        "program": "hip_deployed_shape14_config", "workload": "B1 S100000 D1024 H16 F1024 L2 fp32, default init",
        "official_ratio_rtol0.02_atol0.002": round(ratio, 4), "official_passed": bool(ratio <= 1.0),
        "max_abs": round(errors.max_abs, 6), "mean_abs": round(errors.mean_abs, 7)}
    del outputs, shape14_x
    c, r = summarize_errors(candidate, exact), summarize_errors(reference_path, exact)
    strict = summarize_errors(candidate, reference_path)
    result = {
        "what": "B=1 S=100000 forward of the timed weights: HIP program vs the portable program (bf16, fp32)",
        "passed": summary_no_less_accurate(c, r),
        "candidate_vs_fp32": {"max_abs": round(c.max_abs, 5), "mean_abs": round(c.mean_abs, 6),
                              "gate_failures": c.outside},
        "reference_path_vs_fp32": {"max_abs": round(r.max_abs, 5), "mean_abs": round(r.mean_abs, 6),
                                   "gate_failures": r.outside},
        "candidate_vs_reference_path": {"max_abs": round(strict.max_abs, 5), "gate_failures": strict.outside,
                                        "elements": strict.total},
        "gate_ratio_2e-2_1e-2": round(gate_ratio(candidate, reference_path, atol=2e-2, rtol=1e-2), 4),
        "official_ratio_rtol0.02_atol0.002": round(
            gate_ratio(candidate, reference_path, atol=0.002, rtol=0.02), 4),
        "fp32_io": {
            "what": "fp32 model with fp16 projections and the HIP fp16 attention, B=1 S=100000, against the "
                    "fp32 portable program under the official rule: the timed weights under the reference's "
                    "deployed program shape (hip_deployed_shape14_config: fp32 FFN output projection, HIP fp32 "
                    "norms) and with fp16 branches throughout (hip_mixed_streamed_config: HIP mixed norms); and "
                    "the reference's own Shape 14 (F=1024, default init) under hip_deployed_shape14_config",
            **fp32_io,
            "reference_ratio": 0.2816,
            "reference_ratio_source": "the reference's Triton program, fp32 I/O with fp16 internals, F=1024, "
                                      "default init, RTX 4080 (result/20260831T083857.848038Z/"
                                      "final_performance.json:414)",
        },
    }
    del candidate, reference_path, exact
    torch.cuda.empty_cache()
    ratios = ", ".join(f"{name} {entry['official_ratio_rtol0.02_atol0.002']:.4f}" for name, entry in fp32_io.items())
    log(f"semantic check: passed={result['passed']} candidate max_abs {c.max_abs:.4g} vs reference path "
        f"{r.max_abs:.4g} (against fp32); fp32 I/O official ratios {ratios}")
    return result


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=3)
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-check", action="store_true", help="skip the in-run B=1 semantic check")
    parser.add_argument("--no-resident", action="store_true",
                        help="skip the C2 / C4 latency and the CPU figures of the other configurations")
    parser.add_argument("--cpu-full-layer", action="store_true",
                        help="time every query block of the CPU layer at S=100000 (about two minutes)")
    parser.add_argument("--no-config3", action="store_true",
                        help="skip the operator-alone figures (e.g. for a kernel trace of the forward alone)")
    parser.add_argument("--kernel", choices=("attention", "norm", "copy", "linear", "linear-torch", "gelu", "gelu-torch",
                                             "qkv", "qkv-torch", "boundary", "boundary-torch", "boundary-ffn",
                                             "boundary-ffn-torch", "attention-c3", "norm-c3", "attention-c4"),
                        help="run one kernel alone at the per-chunk shape (profiling)")
    parser.add_argument("--repeat", type=int, default=3, help="launches for --kernel")
    parser.add_argument("--launch", type=lambda text: tuple(int(x) for x in text.split(",")),
                        help="--kernel attention-c3: one launch BLOCK_M,WARPS,STAGES; norm-c3: ROWS,WARPS")
    parser.add_argument("--data", choices=("random", "constant"), default="random",
                        help="--kernel attention inputs: N(0,1) or one constant value (power/clock probe)")
    parser.add_argument("--resident", choices=tuple(RESIDENT_SHAPES),
                        help="time one resident configuration's forward alone (profiling)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU only: the long-sequence workload is "
            "data-parallel over independent sequences, so N GPUs would each run "
            "batch/N sequences with no exchange; this build runs on one GPU.",
            file=sys.stderr,
        )
        return 2
    if args.steps <= 0 or args.warmup < 0:
        raise SystemExit("--steps must be positive and --warmup non-negative")
    if args.kernel in ("attention-c3", "norm-c3"):
        return config3_alone(args.kernel, max(1, args.repeat), None if args.launch is None else [args.launch])
    if args.kernel is not None:
        return kernel_alone(args.kernel, max(1, args.repeat), args.data)
    if args.resident is not None:
        print(json.dumps(resident_latency(RESIDENT_SHAPES[args.resident])), flush=True)
        return 0

    # The operators alone first: directly after the forward the chip runs hot
    # and its clock is lower (attention 114 us there against ~102 us here).
    config3 = None if args.no_config3 else config3_summary()
    gpu = gpu_benchmark(args.steps, args.warmup, check=not args.no_check)
    resident = None
    if not args.no_resident:
        resident = {name: resident_latency(shape, graph=(name == "c2")) for name, shape in RESIDENT_SHAPES.items()}
        log(f"resident: C2 {resident['c2']['median_ms']} ms, C4 {resident['c4']['median_ms']} ms (median)")
    threads, affinity, quota = _cpu_cores()
    baseline = None
    cpu_other = None
    if not args.no_cpu_baseline:
        long_sequence = cpu_long_sequence(threads, full_layer=args.cpu_full_layer)
        baseline = {
            "value": long_sequence["forward_ms"],
            "unit": "ms",
            "cores": threads,
            "kind": "port",
            "sample": long_sequence["sample"],
            # a layer of one sequence: measured in full with --cpu-full-layer,
            # otherwise its attention scaled from the timed query blocks
            ("measured_layer_ms" if long_sequence["layer_is_measured"] else "layer_ms_from_sampled_blocks"):
                long_sequence["layer_ms"],
            "attention_blocks_timed": long_sequence["attention_blocks_timed"],
            "attention_blocks": long_sequence["attention_blocks"],
            "forward_is_extrapolated": True,
            "affinity_cpus": affinity,
            "cgroup_cpu_quota": quota,
        }
        log(f"cpu baseline: layer {long_sequence['layer_ms'] / 1e3:.1f} s "
            f"({'measured' if long_sequence['layer_is_measured'] else 'attention from sampled blocks'}), forward "
            f"{baseline['value'] / 1e3:.0f} s extrapolated, {threads} threads")
        if not args.no_resident:
            cpu_other = cpu_configs(threads)
    achieved = gpu["attention_tflops"]
    traffic = measured_traffic()
    record = {
        "metric": METRIC,
        "value": round(gpu["ms_per_step"], 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["ms_per_step"], 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "long-sequence streamed forward (BASELINE configs[4])",
            "batch": WORKLOAD["batch"],
            "seq_len": WORKLOAD["seq_len"],
            "d_model": WORKLOAD["d_model"],
            "heads": WORKLOAD["heads"],
            "head_dim": WORKLOAD["d_model"] // WORKLOAD["heads"],
            "ffn_dim": WORKLOAD["ffn_dim"],
            "layers": WORKLOAD["layers"],
            "microbatch": WORKLOAD["microbatch"],
            "chunks": WORKLOAD["batch"] // WORKLOAD["microbatch"],
            "config_id": gpu["config_id"],
        },
        "attention": {
            "tflops": round(achieved, 1),
            "pct_mfma_peak": round(100 * achieved / PEAK_BF16_TFLOPS, 2),
            "ms_per_launch": round(gpu["attention_ms_per_launch"], 3),
            "launches_per_step": gpu["attention_launches_per_step"],
            "share_of_step": round(gpu["attention_share_of_step"], 4),
        },
        "norm": {
            "gbs": round(gpu["norm_gbs"], 1),
            "pct_hbm_peak": round(100 * gpu["norm_gbs"] / PEAK_HBM_GBS, 2),
            "us_per_launch": round(gpu["norm_us_per_launch"], 2),
            "bytes_per_launch": int(gpu["norm_bytes_per_launch"]),
        },
        "model_tflops": round(gpu["model_flops"] / (gpu["ms_per_step"] * 1e-3) / 1e12, 1),
        "peak_hbm_bytes_per_chunk": gpu["peak_hbm_bytes_per_chunk"],
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": baseline,
        "semantic_check": gpu.get("semantic_check"),
        "config3": config3,
        "resident_gpu": resident,
        "cpu_configs": cpu_other,
    }
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
