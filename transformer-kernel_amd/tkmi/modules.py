"""Configuration record and parameter tree of the transformer (no compute).

``OptimizedTransformer`` must be a drop-in for the reference harness, whose
strict ``load_state_dict`` (src/torch_transformer_benchmark.py:203-213)
needs the reference's exact parameter names and shapes, and whose seeded
construction (``torch.manual_seed`` then the constructor, :683,690) needs the
same RNG consumption order.  These classes hold exactly that tree:

    layers.{i}.norm1, .attention.{q,k,v,out}_proj, .norm2, .ffn_in, .ffn_out
    final_norm

built in the reference's order (src/torch_transformer_benchmark.py:62-75,
125-132, 148-160).  They carry no forward computation: the fp32 eager
baseline is not part of this package, and ``OptimizedTransformer.forward``
runs entirely on the HIP kernels.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch.nn as nn


@dataclass(frozen=True)
class TransformerConfig:
    """Shape record (src/torch_transformer_benchmark.py:29-56)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by num_heads ({self.num_heads})"
            )
        if self.ffn_dim <= 0:
            raise ValueError("ffn_dim must be positive")
        if self.num_layers <= 0:
            raise ValueError("num_layers must be positive")


class BaselineSelfAttention(nn.Module):
    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)


class BaselineTransformerBlock(nn.Module):
    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = BaselineSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)


class BaselineTransformer(nn.Module):
    """Parameter tree of the reference model; subclasses supply ``forward``."""

    def __init__(self, config) -> None:
        super().__init__()
        self.config = config
        self.layers = nn.ModuleList(
            [
                BaselineTransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
                for _ in range(config.num_layers)
            ]
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x, valid_token_mask=None):  # pragma: no cover - interface only
        raise NotImplementedError(
            "tkmi.BaselineTransformer is the parameter tree only; use "
            "tkmi.OptimizedTransformer for the forward pass"
        )
