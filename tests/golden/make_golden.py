"""Write the numeric golden vectors that pin the CPU oracle.

Each vector is computed by a route independent of the oracle's own code:

* c1_forward.npz -- BASELINE config 1 (B2 S128 D256 H4 F1024 L2, causal),
  PyTorch default init under torch.manual_seed(1234) in the official module
  construction order, input torch.Generator seed 1234.  The forward is
  evaluated in float64 with library routines (F.scaled_dot_product_attention
  with is_causal=True, F.layer_norm, exact F.gelu, F.linear), not with the
  oracle's explicit masked-softmax order.
* tiny_attention.npz -- causal attention of a [1, 2, 7, 4] case by scalar
  Python loops in float64.
* tiny_layer_norm.npz -- residual add + LayerNorm of 3 rows of width 8 by
  scalar Python loops in float64.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

HERE = Path(__file__).resolve().parent
B, S, D, H, FFN, L = 2, 128, 256, 4, 1024, 2


def c1_weights(seed: int) -> dict[str, torch.Tensor]:
    torch.manual_seed(seed)
    state = {}
    for i in range(L):
        p = f"layers.{i}."
        mods = [
            ("norm1", nn.LayerNorm(D)),
            ("attention.q_proj", nn.Linear(D, D)),
            ("attention.k_proj", nn.Linear(D, D)),
            ("attention.v_proj", nn.Linear(D, D)),
            ("attention.out_proj", nn.Linear(D, D)),
            ("norm2", nn.LayerNorm(D)),
            ("ffn_in", nn.Linear(D, FFN)),
            ("ffn_out", nn.Linear(FFN, D)),
        ]
        for name, module in mods:
            state[p + name + ".weight"] = module.weight.detach().clone()
            state[p + name + ".bias"] = module.bias.detach().clone()
    final = nn.LayerNorm(D)
    state["final_norm.weight"] = final.weight.detach().clone()
    state["final_norm.bias"] = final.bias.detach().clone()
    return state


def c1_forward_float64(state: dict[str, torch.Tensor], x: torch.Tensor) -> torch.Tensor:
    w = {k: v.double() for k, v in state.items()}
    x = x.double()

    def lin(t, name):
        return F.linear(t, w[name + ".weight"], w[name + ".bias"])

    def ln(t, name):
        return F.layer_norm(t, (D,), w[name + ".weight"], w[name + ".bias"], 1e-5)

    for i in range(L):
        p = f"layers.{i}."
        h = ln(x, p + "norm1")
        q, k, v = (lin(h, p + f"attention.{n}_proj").view(B, S, H, D // H).transpose(1, 2) for n in "qkv")
        ctx = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + lin(ctx.transpose(1, 2).reshape(B, S, D), p + "attention.out_proj")
        x = x + lin(F.gelu(lin(ln(x, p + "norm2"), p + "ffn_in"), approximate="none"), p + "ffn_out")
    return ln(x, "final_norm")


def tiny_attention() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(7)
    q, k, v = (rng.standard_normal((1, 2, 7, 4)) for _ in range(3))
    out = np.zeros_like(q)
    scale = 1 / math.sqrt(4)
    for b in range(1):
        for h in range(2):
            for i in range(7):
                scores = [sum(q[b, h, i, d] * k[b, h, j, d] for d in range(4)) * scale for j in range(i + 1)]
                m = max(scores)
                e = [math.exp(s - m) for s in scores]
                total = sum(e)
                for d in range(4):
                    out[b, h, i, d] = sum(e[j] * v[b, h, j, d] for j in range(i + 1)) / total
    return {"q": q, "k": k, "v": v, "out": out}


def tiny_layer_norm() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(11)
    value, update = rng.standard_normal((3, 8)), rng.standard_normal((3, 8))
    weight, bias = 1 + 0.5 * rng.standard_normal(8), 0.5 * rng.standard_normal(8)
    out = np.zeros((3, 8))
    for r in range(3):
        row = [value[r, c] + update[r, c] for c in range(8)]
        mean = sum(row) / 8
        var = sum((t - mean) ** 2 for t in row) / 8
        for c in range(8):
            out[r, c] = (row[c] - mean) / math.sqrt(var + 1e-5) * weight[c] + bias[c]
    return {"value": value, "update": update, "weight": weight, "bias": bias, "out": out}


def main() -> None:
    state = c1_weights(1234)
    generator = torch.Generator().manual_seed(1234)
    x = torch.randn(B, S, D, generator=generator)
    out = c1_forward_float64(state, x)
    np.savez_compressed(
        HERE / "c1_forward.npz",
        x=x.numpy(),
        out=out.float().numpy(),
        weight_sums=np.array([float(state[k].double().sum()) for k in sorted(state)]),
        weight_names=np.array(sorted(state)),
    )
    np.savez_compressed(HERE / "tiny_attention.npz", **tiny_attention())
    np.savez_compressed(HERE / "tiny_layer_norm.npz", **tiny_layer_norm())
    print("written to", HERE)


if __name__ == "__main__":
    main()
