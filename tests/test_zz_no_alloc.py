"""tk_small_forward_noalloc: the allocation-free variant of tk_small_forward.

Called through the C ABI on two calls in a row -- C1's shape (B64 S128 L4,
sequences split into 32-row blocks: the scratch's full 1024 hand-off slots)
and then a smaller one (B16 S96 L2) -- its output must equal the allocating
entry point's bit for bit (same kernel, same arithmetic); a split needing
more slots than the scratch holds is rejected with TK_ERR_UNSUPPORTED.
"""

from __future__ import annotations

import pytest
import torch

import tkmi
from tkmi import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _call(fn, opt, x, out):
    w = opt._stacked_weights()
    fn_w, fn_b, fn_eps = opt._final
    lw = opt._weights()[0]
    b, s, d = x.shape
    return getattr(_lib.load(), fn)(
        x.data_ptr(), out.data_ptr(), b, s, d, opt.num_heads, opt.head_dim_padded, opt.config.ffn_dim,
        w["w_qkv"].shape[0], int(opt.config.causal), w["w_qkv"].data_ptr(), w["b_qkv"].data_ptr(),
        w["w_o"].data_ptr(), w["b_o"].data_ptr(), w["w_1"].data_ptr(), w["b_1"].data_ptr(), w["w_2"].data_ptr(),
        w["b_2"].data_ptr(), w["n1_w"].data_ptr(), w["n1_b"].data_ptr(), w["n2_w"].data_ptr(),
        w["n2_b"].data_ptr(), fn_w.data_ptr(), fn_b.data_ptr(), float(lw.n1_eps), float(lw.n2_eps), float(fn_eps),
        float(opt.attn_scale), torch.cuda.current_stream().cuda_stream)


def _error() -> str:
    msg = _lib.load().tk_last_error_string()
    return msg.decode() if msg else ""


def test_noalloc_matches_the_allocating_entry_point():
    for shape in [(64, 128, 128, 4, 128, 4, True), (16, 96, 128, 2, 128, 2, True)]:
        b, s, d = shape[0], shape[1], shape[2]
        opt = tkmi.OptimizedTransformer(tkmi.TransformerConfig(*shape)).to(DEV).eval()
        x = torch.randn(b, s, d, generator=torch.Generator().manual_seed(s + b)).to(DEV)
        want = torch.empty_like(x)
        got = torch.full_like(x, float("nan"))
        with torch.inference_mode():
            opt._weights()
            assert _call("tk_small_forward", opt, x, want) == 0, _error()
            assert _call("tk_small_forward_noalloc", opt, x, got) == 0, _error()
        torch.cuda.synchronize()
        print(f"{shape}: equal={torch.equal(got, want)}", flush=True)
        assert torch.isfinite(want).all()
        assert torch.equal(got, want)


def test_noalloc_rejects_splits_beyond_its_scratch():
    shape = (64, 128, 128, 4, 128, 5, True)  # 64 x 5 x 4 = 1280 hand-off slots
    opt = tkmi.OptimizedTransformer(tkmi.TransformerConfig(*shape)).to(DEV).eval()
    x = torch.randn(64, 128, 128, device=DEV)
    out = torch.empty_like(x)
    with torch.inference_mode():
        opt._weights()
        rc = _call("tk_small_forward_noalloc", opt, x, out)
    assert rc == -2  # TK_ERR_UNSUPPORTED
    assert "static scratch" in _error()
