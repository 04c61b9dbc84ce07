"""Launch-parameter search for the gfx950 HIP programs, feeding the
deployment registry.

The reference selects a program per shape by searching a narrow, explicit
space and publishing the measured winner under the environment fingerprint
(autotune/shape14_search_space.py:25-78 for the streamed workload: tiles x
warps x stages x microbatch; deployment/registry.py for the exact-match
registry).  This module restates that flow for the HIP programs of this
build:

* the space is every attention launch the kernel implements, a few norm
  launches, and the runtime choice of the regime (microbatch size for the
  streamed long-sequence scope; eager or graph replay for resident shapes);
* every candidate is first checked by PlanBuilder (an illegal candidate is
  never timed);
* it is a coordinate search: attention launch, then norm launch, then the FFN
  activation path (hipBLASLt + torch GELU, hipBLASLt + the HIP elementwise
  GELU, the fused HIP Linear + exact-GELU kernel, or the whole FFN fused
  through its residual LayerNorm, where the plan builder accepts them), then
  the QKV path (hipBLASLt packed projection with zero-copy
  views, the HIP projection writing head-major Q / K / V, or that
  projection with the initial LayerNorm fused in), then
  the residual boundary (hipBLASLt output projections
  followed by the HIP residual norm, or the fused HIP Linear + residual +
  LayerNorm boundary where the plan builder accepts it), then runtime, each
  stage keeping the best of the previous ones; a stage replaces the
  current choice only when a candidate is faster by more than ``min_gain``
  (1% by default), because repeated timings of one program differ by a few
  tenths of a percent and a noise-level "win" is not a reason to deploy a
  different program;
* before it is published with ``deployment.registry.publish_deployed_config``
  a winner that differs from the default program must be no less accurate
  than the default program on the same input, both measured against the same
  model run in fp32 on the portable (torch) path: finite, max-abs error within
  1.25x of the default program's (or within 2e-2), mean-abs error within 1.25x
  (+1e-4), and at most 1.25x as many elements outside |err| <= 2e-2 or
  |err| <= 1e-2 |ref| (+1e-4 of the elements); ``autotune.accuracy`` holds
  that rule, which the model-level parity tests share.

Long sequences are timed on a slice of ``timed_sequences`` sequences (the
streamed chunks are identical, so the per-sequence cost carries over); the
registry entry is for the full logical shape.

Usage (from the package directory, on the GPU):

    python -m autotune.hip_launch_search --workload c5 --registry PATH [--publish]
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import statistics
import sys
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from pathlib import Path

import torch

from autotune.accuracy import no_less_accurate
from solution.config import (
    HIP_GELU_LAUNCH,
    HIP_LINEAR_LAUNCH,
    HIP_MLP_BOUNDARY_LAUNCH,
    HIP_QKV_LAUNCH,
    AttentionLaunchParams,
    ConfigSpec,
    FFNBackend,
    InitialNormBackend,
    NormLaunchParams,
    QKVMaterialization,
    ResidualNormBackend,
    RuntimeBackend,
    hip_config,
    hip_linear_boundary_launch,
)
from solution.plan import ExecutionContext
from solution.plan_builder import HardwareCapabilities, PlanBuilder
from solution.shape14.defaults import hip_streamed_config
from solution.shape14.hip_streaming_dh64 import launch_config_is_valid

# Every (block_m, block_n, num_warps, num_stages) the attention kernel runs.
ATTENTION_LAUNCHES: tuple[AttentionLaunchParams, ...] = tuple(
    AttentionLaunchParams(block_m, 64, warps, stages)
    for block_m in (128, 256, 512)
    for warps in (4, 8)
    for stages in (1, 2, 3)
    if launch_config_is_valid(block_m, 64, warps, stages)
)
NORM_LAUNCHES: tuple[NormLaunchParams, ...] = (
    NormLaunchParams(4, 4),
    NormLaunchParams(8, 8),
    NormLaunchParams(2, 2),
    NormLaunchParams(16, 8),
)
MICROBATCHES: tuple[int, ...] = (1, 2, 4)

# The model configurations of BASELINE.json (2, 4 and 5; bf16):
# batch, seq, width, heads, ffn, layers.
WORKLOADS: dict[str, tuple[int, int, int, int, int, int]] = {
    "c2": (64, 256, 512, 8, 2048, 4),
    "c4": (16, 4096, 2048, 32, 8192, 2),
    "c5": (32, 100000, 1024, 16, 4096, 2),
}


@dataclass(frozen=True)
class SearchShape:
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool = True


@dataclass(frozen=True)
class Measurement:
    config: ConfigSpec
    ms_per_sequence: float


def _runtime_variants(config: ConfigSpec, *, streamed: bool, batch: int) -> list[ConfigSpec]:
    schedule = config.schedule
    if streamed:
        return [
            dataclasses.replace(config, schedule=dataclasses.replace(schedule, microbatch_size=m))
            for m in MICROBATCHES
            if batch % m == 0
        ]
    return [
        dataclasses.replace(config, schedule=dataclasses.replace(schedule, runtime=runtime))
        for runtime in (RuntimeBackend.EAGER, RuntimeBackend.CUDA_GRAPH)
    ]


def _with_attention(config: ConfigSpec, launch: AttentionLaunchParams) -> ConfigSpec:
    return dataclasses.replace(config, schedule=dataclasses.replace(config.schedule, attention_launch=launch))


def _ffn_variants(config: ConfigSpec) -> list[ConfigSpec]:
    """The FFN activation paths: hipBLASLt followed by torch's GELU or by the
    HIP elementwise GELU, the fused HIP Linear + bias + exact-GELU kernel,
    each with its launch, and the whole FFN fused through its residual
    LayerNorm (whose launch is also the residual norms'; legal only at the
    widths that kernel serves)."""

    def with_ffn(backend: FFNBackend, ffn_launch=None, ffn_input_launch=None, residual_norm_launch=None) -> ConfigSpec:
        schedule = dataclasses.replace(config.schedule, ffn_launch=ffn_launch, ffn_input_launch=ffn_input_launch)
        if residual_norm_launch is not None:
            schedule = dataclasses.replace(schedule, residual_norm_launch=residual_norm_launch)
        return dataclasses.replace(
            config, program=dataclasses.replace(config.program, ffn=backend), schedule=schedule
        )

    return [
        with_ffn(FFNBackend.TORCH),
        with_ffn(FFNBackend.HIP_EXACT_GELU, ffn_launch=HIP_GELU_LAUNCH),
        with_ffn(FFNBackend.HIP_LINEAR_EXACT_GELU, ffn_input_launch=HIP_LINEAR_LAUNCH),
        with_ffn(FFNBackend.HIP_FUSED_MLP_BOUNDARY, residual_norm_launch=HIP_MLP_BOUNDARY_LAUNCH),
    ]


def _qkv_variants(config: ConfigSpec) -> list[ConfigSpec]:
    """The QKV paths: hipBLASLt's packed projection viewed as Q / K / V, the
    HIP projection with the head-major epilogue, each with its launch, and
    that projection with layer 0's LayerNorm fused into it (no launch of the
    initial norm's own)."""

    def with_qkv(materialization: QKVMaterialization, launch=None) -> ConfigSpec:
        return dataclasses.replace(
            config,
            program=dataclasses.replace(config.program, qkv_materialization=materialization),
            schedule=dataclasses.replace(config.schedule, qkv_launch=launch),
        )

    native = with_qkv(QKVMaterialization.HIP_NATIVE_BHSD, HIP_QKV_LAUNCH)
    fused_initial_norm = dataclasses.replace(
        native,
        program=dataclasses.replace(native.program, initial_norm=InitialNormBackend.HIP_FUSED_QKV),
        schedule=dataclasses.replace(native.schedule, initial_norm_launch=None),
    )
    return [with_qkv(QKVMaterialization.VIEW), native, fused_initial_norm]


def _boundary_variants(config: ConfigSpec, d_model: int) -> list[ConfigSpec]:
    """The residual boundaries: the current one, and the output projections
    fused into them (with the width's launch; the initial norm keeps its own)."""

    fused = dataclasses.replace(
        config,
        program=dataclasses.replace(config.program, residual_norm=ResidualNormBackend.HIP_LINEAR_FUSED),
        schedule=dataclasses.replace(config.schedule, residual_norm_launch=hip_linear_boundary_launch(d_model)),
    )
    return [config, fused]


def _with_norms(config: ConfigSpec, launch: NormLaunchParams) -> ConfigSpec:
    schedule = dataclasses.replace(
        config.schedule, residual_norm_launch=launch, initial_norm_launch=launch
    )
    return dataclasses.replace(config, schedule=schedule)


class HipLaunchSearch:
    """Coordinate search over the HIP launch space for one model and shape."""

    def __init__(
        self,
        model: torch.nn.Module,
        shape: SearchShape,
        *,
        timed_sequences: int = 4,
        warmup: int = 1,
        repeats: int = 3,
        min_gain: float = 0.01,
        sample_ms: float = 25.0,
        hardware: HardwareCapabilities | None = None,
        log: Callable[[str], None] = lambda text: None,
    ) -> None:
        self.model = model
        self.shape = shape
        self.streamed = shape.seq_len >= 32768  # the model's own streamed scope
        self.timed = min(timed_sequences, shape.batch_size) if self.streamed else shape.batch_size
        self.warmup, self.repeats = warmup, repeats
        self.min_gain, self.sample_ms = min_gain, sample_ms
        self.builder = PlanBuilder()
        self.hardware = hardware
        self.log = log
        self.timings: list[Measurement] = []

    def incumbent(self) -> ConfigSpec:
        return hip_streamed_config() if self.streamed else hip_config()

    def _context(self, config: ConfigSpec, device: torch.device) -> ExecutionContext:
        s = self.shape
        return ExecutionContext(
            batch_size=s.batch_size, seq_len=s.seq_len, d_model=s.d_model, num_heads=s.num_heads,
            causal=s.causal, device=device, dtype=torch.bfloat16, training=False, grad_enabled=False,
            input_contiguous=True, has_valid_token_mask=False, mask_compatible=True,
            ffn_dim=s.ffn_dim, num_layers=s.num_layers,
        )

    def legal(self, config: ConfigSpec, device: torch.device) -> bool:
        hardware = self.hardware or HardwareCapabilities.detect(device)
        return self.builder.evaluate(config, self._context(config, device), hardware).accepted

    def _time(self, config: ConfigSpec, x: torch.Tensor) -> float:
        """Median over ``repeats`` samples of ms per sequence; each sample runs
        enough forwards back to back to last ``sample_ms`` (a single forward
        of a resident shape is about a millisecond, too short to time alone)."""

        self.model.configure_execution(config=config)

        def sample(count: int) -> float:
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(count):
                self.model(x)
            end.record()
            torch.cuda.synchronize(x.device)
            return start.elapsed_time(end) / count

        with torch.inference_mode():
            for _ in range(self.warmup):
                self.model(x)
            torch.cuda.synchronize(x.device)
            count = max(1, min(64, math.ceil(self.sample_ms / max(sample(1), 1e-3))))
            times = [sample(count) for _ in range(self.repeats)]
        return statistics.median(times) / x.shape[0]

    def _best(self, configs: Sequence[ConfigSpec], x: torch.Tensor, current: ConfigSpec) -> Measurement:
        """The fastest legal candidate; ``current`` (the choice so far) is kept
        unless another candidate beats it by more than ``min_gain``."""

        best: Measurement | None = None
        kept: Measurement | None = None
        for config in configs:
            if not self.legal(config, x.device):
                continue
            ms = self._time(config, x)
            measurement = Measurement(config, ms)
            self.timings.append(measurement)
            launch = config.schedule.attention_launch
            self.log(
                f"{config.config_id[:16]} attention {launch.to_dict() if launch else None} "
                f"norm {config.schedule.residual_norm_launch.to_dict()} ffn {config.program.ffn.value} "
                f"qkv {config.program.qkv_materialization.value} initial norm {config.program.initial_norm.value} "
                f"boundary {config.program.residual_norm.value} runtime "
                f"{config.schedule.runtime.value}/{config.schedule.microbatch_size}: {ms:.5g} ms/sequence"
            )
            if config.config_id == current.config_id:
                kept = measurement
            if best is None or ms < best.ms_per_sequence:
                best = measurement
        if best is None:
            raise RuntimeError("the plan builder rejected every candidate")
        if kept is not None and best.ms_per_sequence >= kept.ms_per_sequence * (1.0 - self.min_gain):
            return kept
        return best

    def run(self, x: torch.Tensor) -> tuple[Measurement, Measurement]:
        """Returns (winner, incumbent) measured on ``x[: timed]``."""

        timed = x[: self.timed].contiguous()
        incumbent = self.incumbent()
        incumbent_ms = self._time(incumbent, timed)
        base = incumbent
        base = self._best([_with_attention(base, launch) for launch in ATTENTION_LAUNCHES], timed, base).config
        base = self._best([_with_norms(base, launch) for launch in NORM_LAUNCHES], timed, base).config
        base = self._best(_ffn_variants(base), timed, base).config
        base = self._best(_qkv_variants(base), timed, base).config
        base = self._best(_boundary_variants(base, self.shape.d_model), timed, base).config
        winner = self._best(
            _runtime_variants(base, streamed=self.streamed, batch=math.gcd(self.shape.batch_size, self.timed)),
            timed,
            base,
        )
        return winner, Measurement(incumbent, incumbent_ms)

    def _fp32_reference(self, sample: torch.Tensor) -> torch.Tensor:
        """The same weights in fp32 on the portable (torch) path."""

        from solution.config import portable_config, portable_streamed_config
        from solution.transformer import UserOptimizedTransformer

        reference = UserOptimizedTransformer(self.model.config)
        reference.load_state_dict(self.model.state_dict())
        reference = reference.to(device=sample.device, dtype=torch.float32).eval()
        reference.configure_execution(
            config=portable_streamed_config() if self.streamed else portable_config()
        )
        with torch.inference_mode():
            return reference(sample.float())

    def agrees_with_incumbent(self, winner: ConfigSpec, x: torch.Tensor) -> bool:
        """Compares on the timed rows (every runtime variant divides them)."""

        incumbent = self.incumbent()
        if winner.config_id == incumbent.config_id:
            return True
        sample = x[: self.timed].contiguous()
        with torch.inference_mode():
            self.model.configure_execution(config=incumbent)
            want = self.model(sample)
            self.model.configure_execution(config=winner)
            got = self.model(sample)
        reference = self._fp32_reference(sample)
        return no_less_accurate(got, want, reference)


def _seeded_model(shape: SearchShape, device: torch.device, seed: int) -> torch.nn.Module:
    """The workload's model in bf16 with seeded Xavier-uniform weights (q, k, v
    separately inside the packed projection), zero biases, LayerNorm 1 / 0."""

    from solution.transformer import UserOptimizedTransformer

    model = UserOptimizedTransformer(shape)
    generator = torch.Generator().manual_seed(seed)

    def xavier(weight: torch.Tensor) -> torch.Tensor:
        out_features, in_features = weight.shape
        bound = math.sqrt(6.0 / (in_features + out_features))
        return (torch.rand(out_features, in_features, generator=generator) * 2 - 1) * bound

    with torch.no_grad():
        for layer in model.layers:
            width = layer.attention.d_model
            packed = layer.attention.qkv_proj.weight
            for part in range(3):
                rows = packed[part * width : (part + 1) * width]
                rows.copy_(xavier(rows))
            for linear in (layer.attention.out_proj, layer.ffn_in, layer.ffn_out):
                linear.weight.copy_(xavier(linear.weight))
            for linear in (layer.attention.qkv_proj, layer.attention.out_proj, layer.ffn_in, layer.ffn_out):
                linear.bias.zero_()
        for module in model.modules():
            if isinstance(module, torch.nn.LayerNorm):
                module.weight.fill_(1.0)
                module.bias.zero_()
    return model.to(device=device, dtype=torch.bfloat16).eval()


def main(argv: Sequence[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description="HIP launch search -> deployment registry")
    parser.add_argument("--workload", choices=sorted(WORKLOADS), required=True)
    parser.add_argument("--registry", type=Path, required=True, help="deployed-config JSON to update")
    parser.add_argument("--publish", action="store_true", help="write the winner into --registry")
    parser.add_argument("--seed", type=int, default=1234)
    parser.add_argument("--timed-sequences", type=int, default=4)
    parser.add_argument("--repeats", type=int, default=3)
    args = parser.parse_args(argv)

    from deployment.environment import EnvironmentFingerprint, ImplementationScope
    from deployment.registry import ShapeFingerprint, publish_deployed_config
    from solution.kernels.hip import load_library

    device = torch.device("cuda", 0)
    load_library()
    batch, seq, width, heads, ffn, layers = WORKLOADS[args.workload]
    shape = SearchShape(batch, seq, width, heads, ffn, layers)
    model = _seeded_model(shape, device, args.seed)
    generator = torch.Generator(device=device).manual_seed(args.seed)
    search = HipLaunchSearch(
        model, shape, timed_sequences=args.timed_sequences, repeats=args.repeats,
        log=lambda text: print(f"[search] {text}", file=sys.stderr, flush=True),
    )
    rows = search.timed
    x = torch.randn(rows, seq, width, generator=generator, device=device, dtype=torch.bfloat16)
    winner, incumbent = search.run(x)
    agrees = search.agrees_with_incumbent(winner.config, x)
    record = {
        "workload": args.workload,
        "shape": dataclasses.asdict(shape),
        "timed_sequences": rows,
        "incumbent": {"config_id": incumbent.config.config_id, "ms_per_sequence": incumbent.ms_per_sequence},
        "winner": {"config_id": winner.config.config_id, "ms_per_sequence": winner.ms_per_sequence,
                   "config": winner.config.to_dict()},
        "candidates": len(search.timings),
        "agrees_with_incumbent": agrees,
        "published": False,
    }
    if args.publish:
        if not agrees:
            print(json.dumps(record))
            raise SystemExit("winner disagrees with the default program; not published")
        scope = ImplementationScope.SHAPE14 if search.streamed else ImplementationScope.RESIDENT
        publish_deployed_config(
            hardware=EnvironmentFingerprint.detect(device, scope=scope),
            shape=ShapeFingerprint(
                batch_size=batch, qkv_dim=width, heads=heads, seq_len=seq, layers=layers, causal=True,
                ffn_dim=ffn, dtype="bfloat16", padding_ratio=0.0, input_scale=1.0,
            ),
            config=winner.config,
            path=args.registry,
        )
        record["published"] = True
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
