"""Fused QKV projection + one-tile attention (tk_qkv_attention).

The fused kernel computes what the layer path computes in two launches --
tk_gemm into a [T, 3*d_model] q|k|v buffer, then the single-tile flash
kernel on its strided views -- with q, k and v kept on chip.  Checked:
  * bit-identical to that two-launch path (same fp32 accumulation, bias in
    fp32, fp16 rounding, same attention arithmetic), causal and not;
  * against the CPU oracle's attention on the fp32 projection rounded to
    fp16, with the harness's rule |d| <= 0.002 or |d| <= 0.02|ref|
    (src/torch_transformer_benchmark.py:309-316);
  * unsupported shapes are refused, and a model forward on a config-2-like
    shape is identical with and without the fused path.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch
import torch.nn.functional as F

from conftest import or_rule_violations, seeded
from oracle import baseline as ob

import tkmi
from tkmi import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
S, HD = 64, 64


def _operands(batch, heads, seed):
    d = heads * HD
    h = seeded(batch * S, d, dtype=torch.float16, seed=seed)
    w = seeded(3 * d, d, seed=seed + 1, scale=d ** -0.5).half()
    b = seeded(3 * d, seed=seed + 2, scale=0.1)
    return h, w, b


@pytest.mark.parametrize("batch,heads", [(2, 8), (4, 3), (6, 1)], ids=["b2h8", "b4h3", "b6h1"])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_qkv_attention_matches_gemm_then_flash(batch, heads, causal):
    h, w, b = (t.to(DEV) for t in _operands(batch, heads, seed=batch * 10 + heads))
    d = heads * HD
    scale = HD ** -0.5
    fused = ops.qkv_attention(h, w, b, batch, S, heads, HD, scale, causal)
    qkv = ops.linear(h, w, b)
    q, k, v = qkv.view(batch, S, 3, heads, HD).permute(2, 0, 3, 1, 4).unbind(0)
    two_step = ops.flash_attention(q, k, v, scale, causal)
    torch.cuda.synchronize()
    assert fused.shape == (batch * S, d)
    assert torch.equal(fused, two_step.view(batch * S, d))


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_qkv_attention_matches_oracle(causal):
    batch, heads = 4, 8
    h, w, b = _operands(batch, heads, seed=77)
    scale = HD ** -0.5
    got = ops.qkv_attention(h.to(DEV), w.to(DEV), b.to(DEV), batch, S, heads, HD, scale, causal).cpu()
    qkv = F.linear(h.float(), w.float(), b).half()  # the fp16 projection both paths attend over
    q, k, v = qkv.view(batch, S, 3, heads, HD).permute(2, 0, 3, 1, 4).unbind(0)
    ref = ob.attention_ref(q.contiguous(), k.contiguous(), v.contiguous(), scale, causal)
    bad, err = or_rule_violations(got.view(batch, S, heads * HD), ref, atol=2e-3, rtol=2e-2)
    assert bad == 0, err


def test_qkv_attention_refuses_unsupported_shapes():
    assert ops.qkv_attention_supported(2, 64, 8, 64)
    assert not ops.qkv_attention_supported(3, 64, 8, 64)   # 192 tokens: not whole 128-row tiles
    assert not ops.qkv_attention_supported(4, 32, 8, 64)   # S != 64
    assert not ops.qkv_attention_supported(4, 64, 4, 128)  # head_dim != 64
    h, w, b = (t.to(DEV) for t in _operands(4, 2, seed=5))
    with pytest.raises(RuntimeError, match="tk_qkv_attention"):
        ops.qkv_attention(h[: 2 * S // 2], w, b, 1, S, 2, HD, 0.125, True)  # batch 1: 64 tokens


def _pair(cfg, seed=1234):
    base = ob.build_model(cfg, seed=seed).eval()
    opt = tkmi.OptimizedTransformer(tkmi.TransformerConfig(**cfg.__dict__))
    ob.copy_model_weights(base, opt, strict=True)
    return base, opt.to(DEV).eval()


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_model_forward_fused_path_identical(causal):
    cfg = ob.TransformerConfig(8, 64, 512, 8, 1024, 2, causal)
    base, opt = _pair(cfg)
    x = torch.randn(8, 64, 512, generator=torch.Generator().manual_seed(11))
    assert opt.settings.qkv_attention
    with torch.inference_mode():
        fused = opt(x.to(DEV))
        opt.settings = replace(opt.settings, qkv_attention=False)
        layered = opt(x.to(DEV))
    with torch.no_grad():
        ref = base(x)
    assert torch.equal(fused, layered)
    res = ob.compare_outputs(ref, fused.cpu())
    assert res.passed, (res.max_abs_error, res.failed_elements)
