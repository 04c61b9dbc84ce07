"""CPU restatement of the official Transformer forward (test infrastructure).

Follows official/torch_transformer_benchmark.py:
  TransformerConfig            :29-56
  BaselineSelfAttention        :59-123   (separate q/k/v projections, dense
                                          scores, causal -inf mask, fp32 softmax
                                          then cast to the input dtype, P @ V)
  BaselineTransformerBlock     :126-145  (pre-LN, x + attn(norm1(x)),
                                          x + ffn_out(gelu(ffn_in(norm2(x)))))
  BaselineTransformer          :148-172  (layers, then final_norm)
  generate_random_case         :234-272  (padding_ratio == 0 branch)
and the query-blocked attention order of
solution/operators/attention/sdpa.py:116-170 for sequences too long for a
dense [S, S] score matrix.

Weights use the official state-dict names
(``layers.{i}.attention.q_proj.weight`` ...), so they load into both the
official model and, through copy_model_weights, into the solution model.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

LAYER_NORM_EPS = 1e-5  # nn.LayerNorm default, used by every official norm


@dataclass(frozen=True)
class TransformerConfig:
    """Restates official/torch_transformer_benchmark.py:29-56."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads", "ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads:
            raise ValueError("d_model must be divisible by num_heads")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads


# ---------------------------------------------------------------------------
# Weights


def _layer_keys(index: int) -> dict[str, str]:
    prefix = f"layers.{index}."
    return {
        "norm1": prefix + "norm1",
        "q": prefix + "attention.q_proj",
        "k": prefix + "attention.k_proj",
        "v": prefix + "attention.v_proj",
        "out": prefix + "attention.out_proj",
        "norm2": prefix + "norm2",
        "ffn_in": prefix + "ffn_in",
        "ffn_out": prefix + "ffn_out",
    }


def default_init_weights(config: TransformerConfig, seed: int) -> dict[str, torch.Tensor]:
    """PyTorch default init in the official construction order.

    ``torch.manual_seed(seed)`` followed by the modules in the order
    BaselineTransformer.__init__ creates them (per layer: norm1, q/k/v/out
    projections, norm2, ffn_in, ffn_out; then final_norm), which consumes the
    global RNG exactly like official/torch_transformer_benchmark.py:683,690.
    """

    torch.manual_seed(seed)
    state: dict[str, torch.Tensor] = {}
    d, f = config.d_model, config.ffn_dim
    for index in range(config.num_layers):
        keys = _layer_keys(index)
        norm1 = nn.LayerNorm(d)
        linears = {name: nn.Linear(d, d) for name in ("q", "k", "v", "out")}
        norm2 = nn.LayerNorm(d)
        ffn_in = nn.Linear(d, f)
        ffn_out = nn.Linear(f, d)
        modules = {"norm1": norm1, **linears, "norm2": norm2, "ffn_in": ffn_in, "ffn_out": ffn_out}
        for name, module in modules.items():
            state[keys[name] + ".weight"] = module.weight.detach().clone()
            state[keys[name] + ".bias"] = module.bias.detach().clone()
    final = nn.LayerNorm(d)
    state["final_norm.weight"] = final.weight.detach().clone()
    state["final_norm.bias"] = final.bias.detach().clone()
    return state


def xavier_init_weights(config: TransformerConfig, seed: int) -> dict[str, torch.Tensor]:
    """Seeded Xavier-uniform projection weights, zero biases, LayerNorm (1, 0).

    The weight initialisation the BASELINE configurations 2-5 name; biases and
    LayerNorm parameters are not specified there, so zeros / ones are used.
    """

    generator = torch.Generator().manual_seed(seed)
    d, f = config.d_model, config.ffn_dim
    state: dict[str, torch.Tensor] = {}

    def xavier(out_features: int, in_features: int) -> torch.Tensor:
        bound = math.sqrt(6.0 / (in_features + out_features))
        return (torch.rand(out_features, in_features, generator=generator) * 2 - 1) * bound

    for index in range(config.num_layers):
        keys = _layer_keys(index)
        for name in ("norm1", "norm2"):
            state[keys[name] + ".weight"] = torch.ones(d)
            state[keys[name] + ".bias"] = torch.zeros(d)
        for name in ("q", "k", "v", "out"):
            state[keys[name] + ".weight"] = xavier(d, d)
            state[keys[name] + ".bias"] = torch.zeros(d)
        state[keys["ffn_in"] + ".weight"] = xavier(f, d)
        state[keys["ffn_in"] + ".bias"] = torch.zeros(f)
        state[keys["ffn_out"] + ".weight"] = xavier(d, f)
        state[keys["ffn_out"] + ".bias"] = torch.zeros(d)
    state["final_norm.weight"] = torch.ones(d)
    state["final_norm.bias"] = torch.zeros(d)
    return state


def generate_input(
    config: TransformerConfig,
    seed: int,
    *,
    dtype: torch.dtype = torch.float32,
    device: str | torch.device = "cpu",
    input_scale: float = 1.0,
) -> torch.Tensor:
    """Restates generate_random_case with padding_ratio 0 (official :242-258)."""

    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    x = torch.randn(
        config.batch_size,
        config.seq_len,
        config.d_model,
        generator=generator,
        device=device,
        dtype=dtype,
    )
    return x * input_scale


# ---------------------------------------------------------------------------
# Attention


def _split_heads(x: torch.Tensor, heads: int) -> torch.Tensor:
    batch, seq, width = x.shape
    return x.view(batch, seq, heads, width // heads).transpose(1, 2).contiguous()


def dense_causal_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float
) -> torch.Tensor:
    """Official op order (official :97-112): QK^T * scale, -inf above the
    diagonal, softmax in fp32, cast to the input dtype, P @ V."""

    seq = q.shape[-2]
    scores = torch.matmul(q, k.transpose(-2, -1)) * scale
    mask = torch.ones((seq, seq), dtype=torch.bool, device=q.device).triu(diagonal=1)
    scores = scores.masked_fill(mask, float("-inf"))
    probs = torch.softmax(scores.float(), dim=-1).to(q.dtype)
    return torch.matmul(probs, v)


def query_block_causal_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    *,
    query_block: int = 128,
) -> torch.Tensor:
    """Query-blocked order of solution/operators/attention/sdpa.py:116-170:
    the same per-row arithmetic as the dense order with [B, H, block, S]
    temporaries (no key-side causal skipping, like the reference)."""

    seq = q.shape[-2]
    return torch.cat(
        [query_block_rows(q, k, v, scale, start, min(start + query_block, seq))
         for start in range(0, seq, query_block)],
        dim=-2,
    )


def query_block_rows(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, start: int, stop: int
) -> torch.Tensor:
    """Query rows [start, stop) in the order of solution/operators/attention/
    sdpa.py:116-170: scores against every key, scale, causal -inf mask, fp32
    softmax cast to the input dtype, then P V.  Every block does the same
    work, whatever its position (no key-side causal skipping)."""

    key_positions = torch.arange(q.shape[-2], device=q.device)
    scores = torch.matmul(q[..., start:stop, :], k.transpose(-2, -1))
    scores.mul_(scale)
    query_positions = torch.arange(start, stop, device=q.device)
    scores.masked_fill_(key_positions[None, :] > query_positions[:, None], float("-inf"))
    probs = torch.softmax(scores.float(), dim=-1).to(q.dtype)
    return torch.matmul(probs, v)


def causal_attention_rows(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, rows: np.ndarray, scale: float
) -> np.ndarray:
    """Exact float64 causal attention of selected query rows of ONE head.

    q, k, v: [S, Dh] arrays; returns [len(rows), Dh].  Row i attends to keys
    0..i.  Cost is O(len(rows) * S * Dh), so the last rows of a 100k-token
    sequence are affordable on the CPU.
    """

    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    out = np.empty((len(rows), q.shape[1]), dtype=np.float64)
    for index, row in enumerate(rows):
        row = int(row)
        scores = k[: row + 1] @ q[row] * scale
        scores -= scores.max()
        weights = np.exp(scores)
        out[index] = weights @ v[: row + 1] / weights.sum()
    return out


# ---------------------------------------------------------------------------
# Model


def _linear(x: torch.Tensor, state: dict[str, torch.Tensor], name: str) -> torch.Tensor:
    return F.linear(x, state[name + ".weight"], state[name + ".bias"])


def _layer_norm(x: torch.Tensor, state: dict[str, torch.Tensor], name: str) -> torch.Tensor:
    return F.layer_norm(
        x, (x.shape[-1],), state[name + ".weight"], state[name + ".bias"], LAYER_NORM_EPS
    )


def cast_state(state: dict[str, torch.Tensor], dtype: torch.dtype) -> dict[str, torch.Tensor]:
    return {name: tensor.to(dtype) for name, tensor in state.items()}


def forward(
    state: dict[str, torch.Tensor],
    x: torch.Tensor,
    config: TransformerConfig,
    *,
    attention: str = "auto",
) -> torch.Tensor:
    """Official forward in the dtype of ``x`` (weights are cast to it).

    ``attention`` selects the dense official order or the query-blocked order
    ("auto" picks query blocks above 4096 tokens).  Causal only, no padding
    mask (every BASELINE configuration is unpadded and causal).
    """

    if not config.causal:
        raise ValueError("the oracle restates the causal configuration only")
    state = cast_state(state, x.dtype)
    heads = config.num_heads
    scale = config.head_dim**-0.5
    use_blocks = attention == "query_block" or (
        attention == "auto" and x.shape[1] > 4096
    )
    attend = query_block_causal_attention if use_blocks else dense_causal_attention
    for index in range(config.num_layers):
        q, k, v = attention_inputs(state, x, index, heads)
        x = layer_output(state, x, attend(q, k, v, scale), index)
    return final_norm(state, x)


def attention_inputs(
    state: dict[str, torch.Tensor], x: torch.Tensor, index: int, heads: int
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Layer ``index`` up to the attention: norm1, then the q, k and v
    projections split into [B, H, S, Dh] (official :98-106)."""

    keys = _layer_keys(index)
    normalized = _layer_norm(x, state, keys["norm1"])
    return tuple(_split_heads(_linear(normalized, state, keys[name]), heads) for name in ("q", "k", "v"))


def layer_output(
    state: dict[str, torch.Tensor], x: torch.Tensor, context: torch.Tensor, index: int
) -> torch.Tensor:
    """Layer ``index`` after the attention: context [B, H, S, Dh] back to
    [B, S, D], out projection and residual, then norm2, FFN with exact GELU
    and residual (official :112-141)."""

    keys = _layer_keys(index)
    batch, seq, width = x.shape
    context = context.transpose(1, 2).contiguous().view(batch, seq, width)
    x = x + _linear(context, state, keys["out"])
    hidden = F.gelu(_linear(_layer_norm(x, state, keys["norm2"]), state, keys["ffn_in"]), approximate="none")
    return x + _linear(hidden, state, keys["ffn_out"])


def final_norm(state: dict[str, torch.Tensor], x: torch.Tensor) -> torch.Tensor:
    """The model's last LayerNorm (official :169)."""

    return _layer_norm(x, state, "final_norm")


__all__ = [
    "LAYER_NORM_EPS",
    "attention_inputs",
    "final_norm",
    "layer_output",
    "TransformerConfig",
    "cast_state",
    "causal_attention_rows",
    "default_init_weights",
    "dense_causal_attention",
    "forward",
    "generate_input",
    "query_block_causal_attention",
    "query_block_rows",
    "xavier_init_weights",
]
