"""Workload definitions and work models (test / measurement infrastructure).

* estimated_model_flops restates benchmarking/shape14_measure.py:36-46
  (L * (2BS^2D [causal] + 8BSD^2 + 4BSDF)).
* causal_attention_flops is the algorithmic count this build reports against
  the MFMA roofline: QK^T and PV over the causal triangle including the
  diagonal, 4 * B * H * Dh * S(S+1)/2 (softmax exponentials not counted).
* residual_norm_bytes is the algorithmic HBM traffic of one fused boundary:
  rows * width * (value + update + residual + normalized bytes) plus the
  affine parameters once.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Workload:
    name: str
    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    dtype: str
    init: str
    microbatch_size: int | None = None


# BASELINE.json "configs", in order.
C1 = Workload("c1_cpu_fp32", 2, 128, 256, 4, 1024, 2, "float32", "default")
C2 = Workload("c2_short_bf16", 64, 256, 512, 8, 2048, 4, "bfloat16", "xavier")
C3_ATTENTION = (8, 16, 2048, 64)  # B, H, S, Dh
C3_NORM = (16384, 1024)           # rows, width
C4 = Workload("c4_mid_bf16", 16, 4096, 2048, 32, 8192, 2, "bfloat16", "xavier")
C5 = Workload("c5_long_bf16", 32, 100000, 1024, 16, 4096, 2, "bfloat16", "xavier", microbatch_size=2)


def estimated_model_flops(
    *, batch: int, seq: int, width: int, ffn: int, layers: int, causal: bool = True
) -> int:
    attention_factor = 2 if causal else 4
    attention = attention_factor * batch * seq * seq * width
    projections = 8 * batch * seq * width * width
    feed_forward = 4 * batch * seq * width * ffn
    return layers * (attention + projections + feed_forward)


def causal_attention_flops(batch: int, heads: int, seq: int, head_dim: int) -> int:
    return 4 * batch * heads * head_dim * (seq * (seq + 1) // 2)


def residual_norm_bytes(
    rows: int, width: int, *, value: int = 2, update: int = 2, residual: int = 2,
    normalized: int = 2, params: int = 2,
) -> int:
    return rows * width * (value + update + residual + normalized) + 2 * width * params


__all__ = [
    "C1",
    "C2",
    "C3_ATTENTION",
    "C3_NORM",
    "C4",
    "C5",
    "Workload",
    "causal_attention_flops",
    "estimated_model_flops",
    "residual_norm_bytes",
]
