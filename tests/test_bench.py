"""bench.py's host-side pieces on the CPU: the algorithmic work it divides
by (checked against a brute-force count and the BASELINE.md figures), the
one-GPU guard, the rule that reports the profiled HBM traffic only for the
attention sources it was measured on, and the latency summary."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def _query(batch, heads, seq, dim):
    return SimpleNamespace(shape=(batch, heads, seq, dim))


def test_attention_flops_count_every_causal_pair_once():
    """4 FLOPs per (query, visible key, head_dim element): QK^T and PV, a
    multiply and an add each; a key is visible to queries at or after it."""

    batch, heads, seq, dim = 2, 3, 37, 8
    pairs = sum(1 for i in range(seq) for j in range(seq) if j <= i)
    assert bench._attention_flops(_query(batch, heads, seq, dim)) == 4 * batch * heads * dim * pairs


def test_attention_flops_match_the_baseline_figures():
    # one C5 chunk-layer (B2 H16 S1e5) and the C3 operator.
    assert bench._attention_flops(_query(2, 16, 100_000, 64)) == pytest.approx(4.0960e13, rel=1e-4)
    assert bench._attention_flops(_query(8, 16, 2048, 64)) == pytest.approx(6.8753e10, rel=1e-4)
    per_step = 2 * 16 * bench._attention_flops(_query(2, 16, 100_000, 64))
    assert per_step == pytest.approx(1.310733e15, rel=1e-5)


def test_norm_bytes_at_the_c5_boundary():
    """value and update read, residual and normalized written, 2 bytes each
    (bf16), plus gamma and beta once: 1.6384e9 B per C5 chunk boundary."""

    rows, width = 200_000, 1024
    value = torch.empty(rows, width, dtype=torch.bfloat16, device="meta")
    update = torch.empty(rows, width, dtype=torch.bfloat16, device="meta")
    weight = torch.empty(width, dtype=torch.bfloat16, device="meta")
    bias = torch.empty(width, dtype=torch.bfloat16, device="meta")
    assert bench._norm_bytes(value, update, weight, bias, 1e-5, torch.bfloat16) == rows * width * 8 + 2 * width * 2
    # mixed stream: fp32 value and residual, bf16 update and normalized
    value32 = torch.empty(rows, width, dtype=torch.float32, device="meta")
    assert bench._norm_bytes(value32, update, None, None, 1e-5, torch.bfloat16) == rows * width * (8 + 2 + 2)


def test_more_than_one_gpu_is_refused_with_a_reason():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                            capture_output=True, text=True, timeout=300)
    assert result.returncode == 2
    assert "one GPU" in result.stderr
    assert result.stdout == ""


def test_traffic_is_reported_only_for_the_profiled_sources(tmp_path, monkeypatch):
    digest = bench.attention_source_digest()
    assert len(digest) == 16
    profile = tmp_path / "traffic.md"
    monkeypatch.setattr(bench, "TRAFFIC_PROFILE", profile)
    assert bench.measured_traffic() is None  # no profile
    profile.write_text(f"notes\n\nsource_digest = {digest}\ntraffic_bytes_per_launch = 11000000000\n")
    assert bench.measured_traffic() == 11e9
    profile.write_text("source_digest = 0000000000000000\ntraffic_bytes_per_launch = 11000000000\n")
    assert bench.measured_traffic() is None  # measured on other kernel source
    profile.write_text(f"source_digest = {digest}\n")
    assert bench.measured_traffic() is None  # no figure


def test_the_digest_follows_the_attention_sources(tmp_path, monkeypatch):
    sources = []
    for index, path in enumerate(bench.ATTENTION_SOURCES):
        copy = tmp_path / f"{index}_{path.name}"
        copy.write_bytes(path.read_bytes())
        sources.append(copy)
    monkeypatch.setattr(bench, "ATTENTION_SOURCES", tuple(sources))
    before = bench.attention_source_digest()
    assert before == bench.attention_source_digest()
    sources[0].write_bytes(sources[0].read_bytes() + b"\n// edited\n")
    assert bench.attention_source_digest() != before


def test_latency_summary_counts_slow_calls_per_round_position():
    repeats = 20
    samples = [1.0] * (2 * repeats)
    samples[3] = 2.0  # slow call early in round 0
    samples[repeats + 15] = 1.5  # slow call late in round 1
    summary = bench._latency_summary(samples, repeats)
    assert summary["median_ms"] == 1.0
    assert summary["max_ms"] == 2.0
    assert summary["calls_over_1.1x_median"] == 2
    assert summary["of_them_in_first_10_of_a_round"] == 1
    assert summary["p90_ms"] == pytest.approx(1.0)
    json.dumps(summary)


def test_percentile_interpolates_between_ranks():
    assert bench._percentile([4.0, 1.0, 3.0, 2.0], 0.5) == pytest.approx(2.5)
    assert bench._percentile([5.0], 0.9) == 5.0
    assert bench._percentile([1.0, 2.0, 3.0, 4.0, 5.0], 0.9) == pytest.approx(4.6)
