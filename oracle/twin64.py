"""Independent float64 twin of the transformer forward -- TEST INFRASTRUCTURE ONLY.

Written from the equations of the pre-LN block (reference
src/torch_transformer_benchmark.py:85-172) with explicit float64 tensor
arithmetic and no ``torch.nn`` modules, so that a slip in the fp32 oracle
(a dropped bias, a transposed weight, a wrong mask direction, a misplaced
scale) shows up as a disagreement far above fp32 rounding noise.

    LN(x)      = (x - mean) / sqrt(var_pop + eps) * w + b
    attn(h)    = softmax(mask((h Wq^T + bq)_h (h Wk^T + bk)_h^T * hd^-0.5)) (h Wv^T + bv)_h
    block(x)   = x + attn(LN1 x) Wo^T + bo ;  x + W2 gelu(W1 LN2 x + b1) + b2
    out        = LNf(block_L(...block_1(x)))
"""

from __future__ import annotations

import math
from typing import Dict

import torch


def _ln(x, w, b, eps):
    mean = x.sum(-1, keepdim=True) / x.shape[-1]
    c = x - mean
    var = (c * c).sum(-1, keepdim=True) / x.shape[-1]
    return c / torch.sqrt(var + eps) * w + b


def _gelu(x):
    # 0.5 x (1 + erf(x / sqrt 2)) evaluated elementwise with math.erf
    flat = x.reshape(-1).tolist()
    e = torch.tensor([math.erf(v / math.sqrt(2.0)) for v in flat], dtype=torch.float64)
    return 0.5 * x * (1.0 + e.view_as(x))


def _softmax_rows(s):
    m = s.max(dim=-1, keepdim=True).values
    e = torch.exp(s - m)
    return e / e.sum(-1, keepdim=True)


def forward64(state: Dict[str, torch.Tensor], config, x: torch.Tensor, eps: float = 1e-5):
    """float64 forward from a state_dict; dense mask only.  x: [B, S, D]."""
    sd = {k: v.detach().to(torch.float64) for k, v in state.items()}
    x = x.to(torch.float64)
    b, s, d = x.shape
    nh = config.num_heads
    hd = d // nh
    scale = hd ** -0.5
    future = torch.ones(s, s, dtype=torch.bool).triu(1)
    for i in range(config.num_layers):
        p = f"layers.{i}."
        h = _ln(x, sd[p + "norm1.weight"], sd[p + "norm1.bias"], eps)
        proj = {}
        for name in ("q", "k", "v"):
            w = sd[p + f"attention.{name}_proj.weight"]
            bias = sd[p + f"attention.{name}_proj.bias"]
            proj[name] = (h @ w.T + bias).view(b, s, nh, hd).permute(0, 2, 1, 3)
        scores = proj["q"] @ proj["k"].transpose(-1, -2) * scale
        if config.causal:
            scores = scores.masked_fill(future, float("-inf"))
        ctx = _softmax_rows(scores) @ proj["v"]  # [B, H, S, hd]
        ctx = ctx.permute(0, 2, 1, 3).reshape(b, s, d)
        x = x + ctx @ sd[p + "attention.out_proj.weight"].T + sd[p + "attention.out_proj.bias"]
        h = _ln(x, sd[p + "norm2.weight"], sd[p + "norm2.bias"], eps)
        u = _gelu(h @ sd[p + "ffn_in.weight"].T + sd[p + "ffn_in.bias"])
        x = x + u @ sd[p + "ffn_out.weight"].T + sd[p + "ffn_out.bias"]
    return _ln(x, sd["final_norm.weight"], sd["final_norm.bias"], eps)
