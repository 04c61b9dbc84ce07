"""The HIP launch search (autotune/hip_launch_search.py): its space, its
legality filtering and its publication gate (no GPU needed)."""

from __future__ import annotations

import dataclasses

import torch

from autotune.hip_launch_search import (
    ATTENTION_LAUNCHES,
    MICROBATCHES,
    NORM_LAUNCHES,
    WORKLOADS,
    HipLaunchSearch,
    SearchShape,
    _boundary_variants,
    _ffn_variants,
    _qkv_variants,
    _runtime_variants,
    _with_attention,
    _with_norms,
    no_less_accurate,
)
from solution.config import RuntimeBackend, hip_config
from solution.plan_builder import HardwareCapabilities
from solution.shape14.defaults import hip_streamed_config


def _gfx950(**overrides) -> HardwareCapabilities:
    values = dict(
        device_type="cuda", compute_capability=(9, 5), shared_memory_per_block=65536,
        mem_efficient_sdp=False, cudnn_sdp=False, cudnn_available=False, torch_compile=False,
        triton_shape13_attention=False, triton_dh8_attention=False, triton_residual_norm=False,
        triton_mixed_residual_norm=False, triton_initial_norm=False, triton_exact_gelu=False,
        triton_streaming_dh64_attention=False, gcn_arch="gfx950", hip_streaming_dh64_attention=True,
        hip_residual_norm=True, hip_initial_norm=True, hip_exact_gelu=True, hip_linear_exact_gelu=True,
        hip_qkv_native_bhsd=True, hip_linear_residual_norm=True, hip_mlp_residual_norm=True,
    )
    values.update(overrides)
    return HardwareCapabilities(**values)


def test_space_is_every_kernel_launch():
    from solution.kernels.hip import _library

    library = _library.load_library()
    implemented = {
        (m, w, s)
        for m in (64, 128, 256, 512, 1024)
        for w in (2, 4, 8)
        for s in (1, 2, 3, 4)
        if library.sah_causal_attention_launch_supported(m, 64, w, s)
    }
    assert {(l.block_m, l.num_warps, l.num_stages) for l in ATTENTION_LAUNCHES} == implemented


def test_every_candidate_of_the_long_sequence_space_is_legal():
    shape = SearchShape(*WORKLOADS["c5"])
    search = HipLaunchSearch(torch.nn.Identity(), shape, hardware=_gfx950())
    assert search.streamed and search.timed == 4
    device = torch.device("cuda")
    base = search.incumbent()
    assert base == hip_streamed_config()
    for launch in ATTENTION_LAUNCHES:
        assert search.legal(_with_attention(base, launch), device), launch
    for launch in NORM_LAUNCHES:
        assert search.legal(_with_norms(base, launch), device), launch
    variants = _runtime_variants(base, streamed=True, batch=4)
    assert [v.schedule.microbatch_size for v in variants] == list(MICROBATCHES)
    assert all(search.legal(v, device) for v in variants)


def test_resident_space_offers_eager_and_graph_replay():
    shape = SearchShape(*WORKLOADS["c2"])
    search = HipLaunchSearch(torch.nn.Identity(), shape, hardware=_gfx950())
    assert not search.streamed and search.timed == 64 and search.incumbent() == hip_config()
    variants = _runtime_variants(hip_config(), streamed=False, batch=64)
    assert [v.schedule.runtime for v in variants] == [RuntimeBackend.EAGER, RuntimeBackend.CUDA_GRAPH]
    assert all(search.legal(v, torch.device("cuda")) for v in variants)
    # an attention launch the plan builder rejects is never timed: wrong head count
    wide = dataclasses.replace(shape, num_heads=4)
    assert not HipLaunchSearch(torch.nn.Identity(), wide, hardware=_gfx950()).legal(
        hip_config(), torch.device("cuda")
    )


def test_publication_gate():
    generator = torch.Generator().manual_seed(0)
    exact = torch.randn(2, 64, 128, generator=generator) * 3
    # two 16-bit programs: each carries its own accumulated rounding noise
    incumbent = (exact + 0.01 * torch.randn(exact.shape, generator=generator)).to(torch.bfloat16)
    other = (exact + 0.01 * torch.randn(exact.shape, generator=generator)).to(torch.bfloat16)
    assert no_less_accurate(incumbent, incumbent, exact)
    assert no_less_accurate(other, incumbent, exact)
    wrong = other.float().clone()
    wrong.view(-1)[: wrong.numel() // 100] += 0.5  # 1% of the elements far off
    assert not no_less_accurate(wrong.to(torch.bfloat16), incumbent, exact)
    nan = other.float().clone()
    nan.view(-1)[3] = float("nan")
    assert not no_less_accurate(nan.to(torch.bfloat16), incumbent, exact)
    # a dropped term: every element off by a little more than the noise
    biased = (exact + 0.05).to(torch.bfloat16)
    assert not no_less_accurate(biased, incumbent, exact)


def test_a_stage_keeps_the_current_choice_unless_a_candidate_is_clearly_faster():
    shape = SearchShape(*WORKLOADS["c5"])
    search = HipLaunchSearch(torch.nn.Identity(), shape, hardware=_gfx950())
    base = search.incumbent()
    candidates = [_with_attention(base, launch) for launch in ATTENTION_LAUNCHES]
    current = next(c for c in candidates if c.config_id == base.config_id)
    x = torch.zeros(4, 1)
    search.legal = lambda config, device: True

    def timings(table):
        search._time = lambda config, _x: table.get(config.config_id, 100.0)

    # a 0.5% "win" is noise: the current choice stays
    timings({current.config_id: 50.0, candidates[0].config_id: 49.75})
    assert search._best(candidates, x, current).config == current
    # a 5% win replaces it
    timings({current.config_id: 50.0, candidates[0].config_id: 47.5})
    assert search._best(candidates, x, current).config == candidates[0]
    # when the current choice is not among the candidates the fastest wins
    timings({candidates[1].config_id: 10.0})
    assert search._best(candidates[:3], x, hip_config()).config == candidates[1]


def test_ffn_stage_offers_hipblaslt_and_the_fused_kernel():
    from solution.config import FFNBackend

    shape = SearchShape(*WORKLOADS["c5"])
    search = HipLaunchSearch(torch.nn.Identity(), shape, hardware=_gfx950())
    base = search.incumbent()
    variants = _ffn_variants(base)
    assert [v.program.ffn for v in variants] == [
        FFNBackend.TORCH, FFNBackend.HIP_EXACT_GELU, FFNBackend.HIP_LINEAR_EXACT_GELU,
        FFNBackend.HIP_FUSED_MLP_BOUNDARY,
    ]
    assert variants[1] == base  # the default program is one of them
    device = torch.device("cuda")
    assert all(search.legal(v, device) for v in variants[:3])
    # the fused MLP boundary serves widths 128 and 256 only: offered, never timed here
    assert not search.legal(variants[3], device)
    small = HipLaunchSearch(torch.nn.Identity(), SearchShape(8, 128, 256, 4, 1024, 2), hardware=_gfx950())
    small_variants = _ffn_variants(small.incumbent())
    assert small.legal(small_variants[3], device)
    assert small_variants[3].schedule.residual_norm_launch.to_dict() == {"block_rows": 64, "num_warps": 4}
    # without the kernels the HIP variants are rejected, never timed
    no_kernel = HipLaunchSearch(
        torch.nn.Identity(), shape, hardware=_gfx950(hip_exact_gelu=False, hip_linear_exact_gelu=False)
    )
    assert no_kernel.legal(variants[0], device)
    assert not no_kernel.legal(variants[1], device) and not no_kernel.legal(variants[2], device)


def test_qkv_stage_offers_views_the_native_layout_kernel_and_the_fused_initial_norm():
    from solution.config import HIP_QKV_LAUNCH, InitialNormBackend, QKVMaterialization

    for workload in ("c2", "c4", "c5"):
        shape = SearchShape(*WORKLOADS[workload])
        search = HipLaunchSearch(torch.nn.Identity(), shape, hardware=_gfx950())
        base = search.incumbent()
        variants = _qkv_variants(base)
        assert [v.program.qkv_materialization for v in variants] == [
            QKVMaterialization.VIEW, QKVMaterialization.HIP_NATIVE_BHSD, QKVMaterialization.HIP_NATIVE_BHSD,
        ]
        assert [v.program.initial_norm for v in variants] == [
            InitialNormBackend.HIP, InitialNormBackend.HIP, InitialNormBackend.HIP_FUSED_QKV,
        ]
        assert variants[0] == base  # the default program is one of them
        assert variants[1].schedule.qkv_launch == variants[2].schedule.qkv_launch == HIP_QKV_LAUNCH
        assert variants[2].schedule.initial_norm_launch is None
        device = torch.device("cuda")
        assert all(search.legal(v, device) for v in variants), workload
    # without the kernel the native variants are rejected, never timed
    no_kernel = HipLaunchSearch(torch.nn.Identity(), shape, hardware=_gfx950(hip_qkv_native_bhsd=False))
    assert no_kernel.legal(variants[0], device)
    assert not no_kernel.legal(variants[1], device) and not no_kernel.legal(variants[2], device)


def test_boundary_stage_offers_the_fused_linear_boundary_where_it_exists():
    from solution.config import ResidualNormBackend, hip_linear_boundary_launch

    device = torch.device("cuda")
    for workload, legal in (("c2", True), ("c5", True), ("c4", False)):
        shape = SearchShape(*WORKLOADS[workload])
        search = HipLaunchSearch(torch.nn.Identity(), shape, hardware=_gfx950())
        base = search.incumbent()
        variants = _boundary_variants(base, shape.d_model)
        assert variants[0] == base
        fused = variants[1]
        assert fused.program.residual_norm is ResidualNormBackend.HIP_LINEAR_FUSED
        assert fused.schedule.residual_norm_launch == hip_linear_boundary_launch(shape.d_model)
        assert fused.schedule.initial_norm_launch == base.schedule.initial_norm_launch
        assert search.legal(fused, device) is legal, workload  # no 2048-wide instantiation
