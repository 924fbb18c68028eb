"""Per-kernel parity on the GPU: libtkmi vs the CPU oracle on the same seeded inputs.

Test matrices follow the reference's own kernel tests:
  * LayerNorm: dims [32, 64, 100, 128, 1024] x residual {none, fp16, fp32}, 48 rows,
    fp32 sum bit-exact, fp16 output within atol 2e-3 / rtol 2e-2
    (src/test_triton_kernels.py:62-117); widths (32, 128, 1024, 33, 100, 768,
    2048) x 257 rows, fp32 out 1e-5, fp16 out 1e-3, sum 1e-6
    (src/test_kernels.py:54-93);
  * attention: ATTN_SHAPES x {causal, full}, strided q/k/v views of the fused
    projection, the [B, S, H*hd] output layout, ragged S in {32, 33, 64, 100}
    (src/test_triton_kernels.py:144-225), at atol 2e-3 / rtol 2e-2.
GEMM tolerances are stated per test: fp32 accumulation on both sides, so the
only difference is accumulation order (~1e-6 rel) plus the fp16 output cast
(<= 2^-11 rel).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from conftest import fp16_excess, or_rule_violations, seeded
from oracle import baseline as ob

import tkmi
from tkmi import _lib, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


# --------------------------------------------------------------------------- #
# LayerNorm
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("d", [32, 64, 100, 128, 1024])
@pytest.mark.parametrize("residual_dtype", [None, torch.float16, torch.float32])
def test_layernorm_reference_matrix(d, residual_dtype):
    rows = 48
    x = seeded(rows, d, seed=d)
    w = seeded(d, seed=d + 1, scale=0.5) + 1.0
    b = seeded(d, seed=d + 2, scale=0.5)
    xg, wg, bg = x.to(DEV), w.to(DEV), b.to(DEV)
    if residual_dtype is None:
        y = ops.ln_fwd(xg, wg, bg, 1e-5, out_dtype=torch.float16)
        expected_sum = x
    else:
        r = seeded(rows, d, dtype=residual_dtype, seed=d + 3)
        expected_sum = x + r.float()
        s, y = ops.add_ln_fwd(xg, r.to(DEV), wg, bg, 1e-5, out_dtype=torch.float16)
        assert torch.equal(s.cpu(), expected_sum)  # the fp32 add is one IEEE op: bit-exact
    ref = ob.layer_norm_ref(expected_sum, w, b, 1e-5, torch.float16)
    assert y.dtype == torch.float16 and y.shape == x.shape
    bad, err = or_rule_violations(y, ref, atol=2e-3, rtol=2e-2)
    assert bad == 0, err


def test_layernorm_fp32_out_is_tight():
    d, rows = 128, 32
    x, r = seeded(rows, d, seed=7), seeded(rows, d, seed=8)
    w, b = seeded(d, seed=9) + 1.0, seeded(d, seed=10)
    _, y = ops.add_ln_fwd(x.to(DEV), r.to(DEV), w.to(DEV), b.to(DEV), 1e-5)
    ref = ob.layer_norm_ref(x + r, w, b, 1e-5)
    torch.testing.assert_close(y.cpu(), ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("cols", [64, 100, 1024])
def test_layernorm_row_mask_zeroes_padded_rows(cols):
    """Final-norm semantics of a padded row (src/torch_transformer_benchmark.py:170-171)."""
    rows = 37
    x = seeded(rows, cols, seed=cols) * 3
    w, b = seeded(cols, seed=cols + 1) + 1.0, seeded(cols, seed=cols + 2)
    valid = torch.rand(rows, generator=torch.Generator().manual_seed(cols)) < 0.5
    ref = ob.layer_norm_ref(x, w, b, 1e-5).masked_fill(~valid[:, None], 0)
    y = ops.ln_fwd(x.to(DEV), w.to(DEV), b.to(DEV), 1e-5, torch.float32, row_valid=valid.to(DEV))
    torch.testing.assert_close(y.cpu(), ref, atol=1e-5, rtol=1e-5)
    assert bool((y.cpu()[~valid] == 0).all())


def test_layernorm_three_dim_and_noncontiguous():
    x = seeded(3, 5, 128, seed=21)
    r = seeded(3, 5, 128, dtype=torch.float16, seed=22)
    w, b = seeded(128, seed=23) + 1.0, seeded(128, seed=24)
    s, y = ops.add_ln_fwd(x.to(DEV), r.to(DEV), w.to(DEV), b.to(DEV), 1e-5)
    assert y.shape == (3, 5, 128) and s.shape == (3, 5, 128)
    torch.testing.assert_close(y.cpu(), ob.layer_norm_ref(x + r.float(), w, b), atol=1e-5, rtol=1e-5)
    x3 = seeded(4, 16, 128, seed=25).transpose(0, 1)
    got = ops.ln_fwd(x3.to(DEV), w.to(DEV), b.to(DEV), 1e-5, torch.float16)
    assert fp16_excess(got, ob.layer_norm_ref(x3, w, b, 1e-5, torch.float16), atol=1e-3) <= 0


@pytest.mark.parametrize("n_cols", [32, 128, 1024, 33, 100, 768, 2048])
def test_layernorm_script_matrix(n_cols):
    rows = 257
    x = seeded(rows, n_cols, seed=n_cols) * 3
    y = seeded(rows, n_cols, dtype=torch.float16, seed=n_cols + 1)
    w, b = seeded(n_cols, seed=n_cols + 2), seeded(n_cols, seed=n_cols + 3)
    xg, yg, wg, bg = x.to(DEV), y.to(DEV), w.to(DEV), b.to(DEV)
    # fp32 out: |d| <= 1e-5; fp16 out: |d| <= max(1e-3, 1 fp16 ulp of the reference)
    for out_dtype, atol in ((torch.float32, 1e-5), (torch.float16, 1e-3)):
        got = ops.ln_fwd(xg, wg, bg, 1e-5, out_dtype)
        want = ob.layer_norm_ref(x, w, b, 1e-5, out_dtype)
        s, h = ops.add_ln_fwd(xg, yg, wg, bg, 1e-5, out_dtype)
        sum_want = x + y.float()
        h_want = ob.layer_norm_ref(sum_want, w, b, 1e-5, out_dtype)
        assert (s.cpu() - sum_want).abs().max() <= 1e-6
        if out_dtype == torch.float32:
            assert (got.cpu() - want).abs().max() <= atol
            assert (h.cpu() - h_want).abs().max() <= atol
        else:
            assert fp16_excess(got, want, atol) <= 0
            assert fp16_excess(h, h_want, atol) <= 0


@pytest.mark.parametrize("cols", [64, 100, 1024])
@pytest.mark.parametrize("y_dtype", [torch.float16, torch.float32])
def test_add_ln_half_x_returns_sum_in_x_dtype(cols, y_dtype):
    """fp16 x: s = x + y is added in fp32 and returned in x's dtype, h = LN of the
    fp32 sum in out_dtype (default x's dtype), as src/fused_kernels.py:196-238
    (s = empty_like(x2) at :216, the sum stored through sum_ptr's element type at
    :143-147, the statistics from the fp32 s at :149-154).  cols 100 takes the
    scalar path."""
    rows = 129
    x = seeded(rows, cols, dtype=torch.float16, seed=cols + 40) * 2
    y = seeded(rows, cols, dtype=y_dtype, seed=cols + 41)
    w, b = seeded(cols, seed=cols + 42, scale=0.5) + 1.0, seeded(cols, seed=cols + 43, scale=0.5)
    xg, yg, wg, bg = x.to(DEV), y.to(DEV), w.to(DEV), b.to(DEV)
    sum32 = x.float() + y.float()
    s, h = ops.add_ln_fwd(xg, yg, wg, bg, 1e-5)
    assert s.dtype == torch.float16 and h.dtype == torch.float16 and s.shape == x.shape
    assert torch.equal(s.cpu(), sum32.half())  # one fp32 add, one rounding: bit-exact
    assert fp16_excess(h, ob.layer_norm_ref(sum32, w, b, 1e-5, torch.float16), 1e-3) <= 0
    s2, h32 = ops.add_ln_fwd(xg, yg, wg, bg, 1e-5, torch.float32)
    assert s2.dtype == torch.float16 and torch.equal(s2.cpu(), s.cpu())
    # the statistics come from the fp32 sum, not from its fp16 rounding
    torch.testing.assert_close(h32.cpu(), ob.layer_norm_ref(sum32, w, b, 1e-5), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("cols", [512, 2048, 4096, 8192])
def test_layernorm_model_widths_no_sum(cols):
    rows = 300
    x, y = seeded(rows, cols, seed=1), seeded(rows, cols, seed=2)
    w, b = seeded(cols, seed=3) + 1, seeded(cols, seed=4)
    s, h = ops.add_ln_fwd(x.to(DEV), y.to(DEV), w.to(DEV), b.to(DEV), 1e-5, torch.float32, write_sum=False)
    assert s is None
    torch.testing.assert_close(h.cpu(), ob.layer_norm_ref(x + y, w, b), atol=1e-5, rtol=1e-5)


# --------------------------------------------------------------------------- #
# GEMM + epilogues
# --------------------------------------------------------------------------- #

GEMM_SHAPES = [  # one or more per tile configuration of the dispatch, direct and K-tail paths
    (512, 384, 128),      # C1 QKV (reduced M): 64x64 tiles
    (1024, 1536, 512),    # C2 QKV (reduced M)
    (1024, 512, 2048),    # C2 FFN-down (reduced M)
    (4096, 4096, 1024),   # 256x256 tiles
    (8192, 4352, 384),    # 544 256x256 tiles: the persistent ping-pong kernel (bias, GELU and residual
                          # epilogues; 2 or 3 tiles per workgroup, the next tile's first K-tile prefetched)
    (4096, 2048, 8192),   # C4 FFN-down (reduced M), long K: 128x128 tiles
    (1000, 200, 72),      # ragged M, N, K
    (77, 300, 8),         # tiny K
    (130, 130, 136),
    (4000, 2100, 128),    # 128x128 tiles with M and N tails
    (12800, 512, 2048),   # 256x128 tiles, three K stages
    (13000, 500, 2056),   # 256x128 tiles, K tail, M and N tails
    (4100, 4200, 1032),   # 256x256 tiles, K tail, M and N tails
    (1, 384, 128),        # one row
    (300, 1, 64),         # one output column
    (200, 150, 100),      # K not a multiple of 8: element loads, zero fill past K
]


def _gemm_inputs(m, n, k, seed=0):
    a = seeded(m, k, seed=seed).half()
    w = (seeded(n, k, seed=seed + 1) / k ** 0.5).half()
    bias = seeded(n, seed=seed + 2) * 0.1
    ref = a.float() @ w.float().T + bias
    return a, w, bias, ref


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("gelu", [False, True])
def test_gemm_bias_and_gelu(m, n, k, gelu):
    a, w, bias, ref = _gemm_inputs(m, n, k)
    if gelu:
        ref = ob.gelu_ref(ref)
    got = ops.linear(a.to(DEV), w.to(DEV), bias.to(DEV), gelu=gelu)
    # fp16 output: |d| <= 1e-3 + 1e-3*|ref| (cast <= 4.9e-4 rel, accumulation order ~1e-6)
    torch.testing.assert_close(got.cpu().float(), ref.half().float(), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_gemm_residual_inplace(m, n, k):
    a, w, bias, ref = _gemm_inputs(m, n, k, seed=3)
    resid = seeded(m, n, seed=9)
    rg = resid.to(DEV)
    out = ops.linear_residual(a.to(DEV), w.to(DEV), bias.to(DEV), rg, out=rg)
    assert out.data_ptr() == rg.data_ptr()
    # fp32 output: accumulation-order differences only
    torch.testing.assert_close(out.cpu(), resid + ref, atol=5e-5, rtol=1e-5)


# 256 x 256 tiles: launches of whole tiles (M, N multiples of 256, K of 128) run
# the ping-pong K loop, others the two-stage loop (or 128 x 128 tiles); per
# output element both accumulate the same MFMA k-steps in the same order, so
# the first M rows of an (M + 8)-row launch equal the whole-tile launch bit for bit.
@pytest.mark.parametrize("m,n,k", [(4096, 4096, 2048), (8192, 8192, 512), (8192, 2048, 4096)])
@pytest.mark.parametrize("epi", ["bias", "gelu", "resid"])
def test_gemm_pingpong_matches_two_stage_loop(m, n, k, epi):
    a, w, bias, ref = _gemm_inputs(m + 8, n, k, seed=31)
    ag, wg, bg = a.to(DEV), w.to(DEV), bias.to(DEV)
    if epi == "resid":
        resid = seeded(m + 8, n, seed=32).to(DEV)
        whole = ops.linear_residual(ag[:m], wg, bg, resid[:m].contiguous())
        ragged = ops.linear_residual(ag, wg, bg, resid)
        want = resid.cpu() + ref
        tol = dict(atol=5e-5, rtol=1e-5)
    else:
        whole = ops.linear(ag[:m], wg, bg, gelu=epi == "gelu")
        ragged = ops.linear(ag, wg, bg, gelu=epi == "gelu")
        want = (ob.gelu_ref(ref) if epi == "gelu" else ref).half().float()
        tol = dict(atol=1e-3, rtol=1e-3)
    assert torch.equal(whole, ragged[:m])
    torch.testing.assert_close(ragged.cpu().float(), want, **tol)


@pytest.mark.parametrize("mode", ["keep", "zero"])
def test_gemm_residual_row_mask(mode):
    """Padded rows of the residual update: the product counts as 0 (keep resid,
    after attention) or the row becomes 0 (after the FFN)."""
    m, n, k = 300, 192, 64
    a, w, bias, ref = _gemm_inputs(m, n, k, seed=12)
    resid = seeded(m, n, seed=13)
    valid = torch.rand(m, generator=torch.Generator().manual_seed(14)) < 0.6
    a[~valid] = float("nan")  # a padded row's input may be non-finite (fully masked attention row)
    code = ops.TK_ROWS_KEEP_RESID if mode == "keep" else ops.TK_ROWS_ZERO
    out = ops.linear_residual(a.to(DEV), w.to(DEV), bias.to(DEV), resid.to(DEV), row_valid=valid.to(DEV),
                              row_mode=code).cpu()
    want = torch.where(valid[:, None], resid + ref, resid if mode == "keep" else torch.zeros_like(resid))
    torch.testing.assert_close(out[valid], want[valid], atol=5e-5, rtol=1e-5)
    assert torch.equal(out[~valid], want[~valid])


@pytest.mark.parametrize("mode", ["keep", "zero", "zero_all"])
def test_gemm_add_layernorm_row_mask(mode):
    m, n, k = 200, 128, 256
    a, w, bias, acc = _gemm_inputs(m, n, k, seed=15)
    resid = seeded(m, n, seed=16) * 2
    lw, lb = seeded(n, seed=17) * 0.3 + 1, seeded(n, seed=18) * 0.3
    valid = torch.rand(m, generator=torch.Generator().manual_seed(19)) < 0.5
    a[~valid] = float("nan")
    code = {"keep": ops.TK_ROWS_KEEP_RESID, "zero": ops.TK_ROWS_ZERO, "zero_all": ops.TK_ROWS_ZERO_ALL}[mode]
    s_ref = torch.where(valid[:, None], resid + acc, resid if mode == "keep" else torch.zeros_like(resid))
    h_ref = ob.layer_norm_ref(s_ref, lw, lb, 1e-5)
    if mode == "zero_all":
        h_ref = h_ref.masked_fill(~valid[:, None], 0)
    sg = torch.empty(m, n, device=DEV)
    h = ops.linear_add_ln(a.to(DEV), w.to(DEV), bias.to(DEV), resid.to(DEV), lw.to(DEV), lb.to(DEV), 1e-5,
                          torch.float32, sum_out=sg, row_valid=valid.to(DEV), row_mode=code)
    torch.testing.assert_close(sg.cpu(), s_ref, atol=5e-5, rtol=1e-5)
    torch.testing.assert_close(h.cpu(), h_ref, atol=1e-4, rtol=1e-4)


def test_gemm_strided_operand():
    a, w, bias, ref = _gemm_inputs(256, 128, 64, seed=5)
    big = torch.zeros(256, 96, dtype=torch.float16)
    big[:, 16:80] = a
    view = big.to(DEV)[:, 16:80]
    got = ops.linear(view, w.to(DEV), bias.to(DEV))
    torch.testing.assert_close(got.cpu().float(), ref.half().float(), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("n", [128, 256, 512])
@pytest.mark.parametrize("m", [64, 1000, 4096])
def test_gemm_add_layernorm_epilogue(m, n):
    k = 2 * n
    a, w, bias, acc = _gemm_inputs(m, n, k, seed=n)
    resid = seeded(m, n, seed=n + 7) * 2
    lw, lb = seeded(n, seed=n + 8) * 0.3 + 1, seeded(n, seed=n + 9) * 0.3
    s_ref = resid + acc
    h_ref = ob.layer_norm_ref(s_ref, lw, lb, 1e-5)
    rg = resid.to(DEV)
    h = ops.linear_add_ln(a.to(DEV), w.to(DEV), bias.to(DEV), rg, lw.to(DEV), lb.to(DEV), 1e-5,
                          torch.float16, sum_out=rg)
    torch.testing.assert_close(rg.cpu(), s_ref, atol=5e-5, rtol=1e-5)
    torch.testing.assert_close(h.cpu().float(), h_ref.half().float(), atol=2e-3, rtol=2e-3)
    h32 = ops.linear_add_ln(a.to(DEV), w.to(DEV), bias.to(DEV), resid.to(DEV), lw.to(DEV), lb.to(DEV),
                            1e-5, torch.float32)
    torch.testing.assert_close(h32.cpu(), h_ref, atol=1e-4, rtol=1e-4)


# --------------------------------------------------------------------------- #
# Attention
# --------------------------------------------------------------------------- #

ATTN_SHAPES = [  # (B, H, S, hd); the reference's shapes (src/test_triton_kernels.py:144-152) first
    (2, 4, 128, 32),
    (2, 16, 64, 8),     # head_dim 8: the element-load kernel on the 16-wide tile
    (1, 1, 64, 128),
    (2, 4, 96, 32),
    (1, 2, 128, 64),
    (1, 4, 32, 16),
    (8, 16, 512, 64),   # 128-row tile path
    (1, 2, 1024, 128),
    (4, 8, 64, 64),     # C2-like: one key tile per head
    (1, 2, 64, 256),
    (2, 3, 700, 256),   # head_dim 256, 4-wave tiles, ragged last tile
    (2, 2, 1, 64),      # one key
    (2, 1, 63, 32),     # one key short of a tile
    (1, 2, 65, 64),     # one key past the first tile
    (1, 2, 129, 64),    # past 128 rows: the long-sequence dispatch
    (1, 2, 129, 128),
]


def _qkv(shape, seed=1):
    return tuple(seeded(*shape, dtype=torch.float16, seed=seed + i) for i in range(3))


@pytest.mark.parametrize("shape", ATTN_SHAPES, ids=lambda s: "b{}h{}s{}d{}".format(*s))
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_flash_attention_matches_reference(shape, causal):
    b, h, s, hd = shape
    q, k, v = _qkv(shape)
    out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal)
    ref = ob.attention_ref(q, k, v, hd ** -0.5, causal)
    assert out.shape == (b, s, h * hd)
    bad, err = or_rule_violations(out, ref, atol=2e-3, rtol=2e-2)
    assert bad == 0, err


def test_flash_attention_strided_qkv_views():
    b, h, s, hd = 2, 4, 128, 32
    qkv = seeded(b, s, 3, h, hd, dtype=torch.float16, seed=42)
    q, k, v = qkv.to(DEV).permute(2, 0, 3, 1, 4).unbind(0)
    assert not q.is_contiguous()
    out = ops.flash_attention(q, k, v, hd ** -0.5, causal=True)
    qc, kc, vc = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    bad, err = or_rule_violations(out, ob.attention_ref(qc, kc, vc, hd ** -0.5, True))
    assert bad == 0, err


def test_flash_attention_output_layout():
    b, h, s, hd = 1, 2, 64, 64
    q, k, v = _qkv((b, h, s, hd), seed=5)
    out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal=True)
    assert out.stride() == (s * h * hd, h * hd, 1)
    bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, True))
    assert bad == 0, err


@pytest.mark.parametrize("s", [32, 33, 64, 100])
def test_flash_attention_ragged_sequence_lengths(s):
    b, h, hd = 1, 2, 32
    q, k, v = _qkv((b, h, s, hd), seed=s)
    for causal in (True, False):
        out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal)
        bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, causal))
        assert bad == 0, (causal, err)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("s", [512, 600, 777, 1000, 1300])
def test_flash_attention_long_ragged(s, hd):
    """Long sequences (the two-group kernel): lengths off the 64-key tile and
    256-row block grid, causal and full."""
    b, h = 1, 2
    q, k, v = _qkv((b, h, s, hd), seed=s + hd)
    for causal in (True, False):
        out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal)
        bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, causal))
        assert bad == 0, (causal, err)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("s", [1024, 1300, 2100])
def test_flash_attention_epoch_loop_is_bit_identical(s, hd):
    """Causal, head_dim 128 (256-row query blocks) and 64 (128-row blocks): the
    key tiles below a query block's diagonal run from a generated asm loop
    (tk_attn_epochs.inc, tk_attn_steps64.inc) when the K/V copy span fits 32-bit
    offsets.  K/V rows 4 MiB apart put the span past 2^31 bytes for every query
    block that would use the loop, so the same values take the compiled steps;
    the loop changes the instruction order, not the arithmetic, so the two
    outputs must agree bit for bit (and both with the reference)."""
    b, h = 1, 1
    q, k, v = _qkv((b, h, s, hd), seed=s)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    compact = ops.flash_attention(qd, kd, vd, hd ** -0.5, True)
    rs = 1 << 21  # fp16 elements between K (and V) rows
    wide_k = torch.zeros(s, rs, dtype=torch.float16, device=DEV)
    wide_v = torch.zeros(s, rs, dtype=torch.float16, device=DEV)
    wide_k[:, :hd] = kd[0, 0]
    wide_v[:, :hd] = vd[0, 0]
    kw, vw = wide_k[:, :hd][None, None], wide_v[:, :hd][None, None]
    assert kw.stride(2) == rs and torch.equal(kw, kd)
    spread = ops.flash_attention(qd, kw, vw, hd ** -0.5, True)
    del wide_k, wide_v
    assert torch.equal(compact, spread)
    bad, err = or_rule_violations(compact, ob.attention_ref(q, k, v, hd ** -0.5, True))
    assert bad == 0, err


@pytest.mark.parametrize("hd,s", [(64, n) for n in (319, 320, 383, 384, 385, 447, 448, 449, 575, 576, 640)]
                         + [(128, n) for n in (575, 576, 639, 640, 641, 767, 768, 769, 832, 1023, 1025)])
def test_flash_attention_epoch_loop_boundaries(hd, s):
    """Causal lengths around the points where the asm steady state's step count
    changes (head_dim 64: 128-row query blocks, steps up to min(q0/64 - 1,
    min(n_kt, S/64) - 3); head_dim 128: 256-row blocks, epochs up to
    min(q0/64, min(n_kt, S/64) - 2)), against the reference."""
    b, h = 1, 2
    q, k, v = _qkv((b, h, s, hd), seed=3 * s + hd)
    out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, True)
    bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, True))
    assert bad == 0, err


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_flash_attention_v_rows_8_byte_aligned(causal):
    """head_dim 128 with V rows only 8-byte aligned: the non-causal body loads V
    8 bytes at a time, the causal bodies copy 16-byte chunks and must not get it
    (such calls take the element-load kernel)."""
    b, h, s, hd = 1, 2, 300, 128
    q, k, v = _qkv((b, h, s, hd), seed=11)
    vbuf = torch.zeros(b, h, s, hd + 8, dtype=torch.float16, device=DEV)
    vbuf[..., 4:4 + hd] = v.to(DEV)
    vv = vbuf[..., 4:4 + hd]
    assert vv.data_ptr() % 16 == 8 and torch.equal(vv.cpu(), v)
    out = ops.flash_attention(q.to(DEV), k.to(DEV), vv, hd ** -0.5, causal)
    bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, causal))
    assert bad == 0, err


@pytest.mark.parametrize("hd", [64, 128])
def test_flash_attention_long_strided_views(hd):
    """q/k/v as strided views of one fused [B, S, 3, H, hd] projection, as the model passes them."""
    b, h, s = 2, 3, 1100
    qkv = seeded(b, s, 3, h, hd, dtype=torch.float16, seed=7)
    q, k, v = qkv.to(DEV).permute(2, 0, 3, 1, 4).unbind(0)
    qc, kc, vc = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    for causal in (True, False):
        out = ops.flash_attention(q, k, v, hd ** -0.5, causal)
        bad, err = or_rule_violations(out, ob.attention_ref(qc, kc, vc, hd ** -0.5, causal))
        assert bad == 0, (causal, err)


@pytest.mark.parametrize("hd", [64, 128])
def test_flash_attention_large_logits(hd):
    """Scores spanning many powers of two: the running max moves often (rescale path)
    and most probabilities underflow."""
    b, h, s = 1, 2, 1024
    q, k, v = _qkv((b, h, s, hd), seed=99)
    # growing query norms along the sequence -> the row max jumps across tiles
    ramp = torch.linspace(0.5, 6.0, s).view(1, 1, s, 1)
    q = (q.float() * ramp).half()
    k = (k.float() * 2.0).half()
    for causal in (True, False):
        out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal)
        bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, causal))
        assert bad == 0, (causal, err)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("slope", [6.0, 24.0])
def test_flash_attention_scores_rising_along_keys(hd, slope):
    """Scores that rise by `slope` (in log2 units) per 64-key tile along the keys, for every
    query row: the running max must move on most tiles (24: every tile's exponentials
    against the old reference overflow fp16, so the head_dim-64 steps that rescale only on
    overflow and the head_dim-128 loop epochs that take the row max only when a row sum
    reaches 128 redo P on every tile; 6: every third tile or so).  Against the reference, and the
    generated loops against the compiled steps bit for bit (K/V rows 4 MiB apart, as in
    test_flash_attention_epoch_loop_is_bit_identical)."""
    b, h, s = 1, 2, 1024
    g = torch.Generator().manual_seed(int(slope) * 7 + hd)
    u = torch.randn(hd, generator=g)
    u = u / u.norm()
    cs = hd ** -0.5 * 1.4426950408889634
    # s_ij * cs = cs * (4 u + noise).(c t_j u + noise) ~ 4 c cs t_j: c for `slope` per tile
    c = slope / (4.0 * cs)
    t = torch.arange(s, dtype=torch.float32) / 64.0
    q = (4.0 * u + 0.1 * torch.randn(b, h, s, hd, generator=g)).half()
    k = (c * t[:, None] * u + torch.randn(b, h, s, hd, generator=g)).half()
    v = torch.randn(b, h, s, hd, generator=g).half()
    assert torch.isfinite(k).all()
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    for causal in (True, False):
        out = ops.flash_attention(qd, kd, vd, hd ** -0.5, causal)
        bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, causal))
        assert bad == 0, (causal, err)
    compact = ops.flash_attention(qd, kd, vd, hd ** -0.5, True)
    rs = 1 << 21
    wide_k = torch.zeros(b * h * s, rs, dtype=torch.float16, device=DEV)
    wide_v = torch.zeros(b * h * s, rs, dtype=torch.float16, device=DEV)
    wide_k[:, :hd] = kd.reshape(-1, hd)
    wide_v[:, :hd] = vd.reshape(-1, hd)
    kw = wide_k.view(b, h, s, rs)[..., :hd]
    vw = wide_v.view(b, h, s, rs)[..., :hd]
    assert kw.stride(2) == rs and torch.equal(kw, kd)
    spread = ops.flash_attention(qd, kw, vw, hd ** -0.5, True)
    del wide_k, wide_v
    assert torch.equal(compact, spread)


def _attention_ref_keymask(q, k, v, scale, causal, key_valid):
    """Baseline order (src/torch_transformer_benchmark.py:97-112) with the key mask of :105-108."""
    scores = torch.matmul(q.float(), k.float().transpose(-2, -1)) * scale
    probs = ob.masked_softmax_ref(scores, causal, key_valid[:, None, None, :])
    b, h, s, hd = q.shape
    return torch.matmul(probs, v.float()).transpose(1, 2).reshape(b, s, h * hd)


@pytest.mark.parametrize("shape", [(2, 4, 128, 32), (3, 2, 100, 64), (2, 2, 700, 128), (1, 2, 1300, 128),
                                   (1, 2, 64, 16),
                                   (1, 2, 300, 256), (2, 1, 64, 256),  # head_dim 256 (generic vector kernel)
                                   (2, 2, 90, 48)],                    # element-load kernel
                         ids=lambda s: "b{}h{}s{}d{}".format(*s))
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_flash_attention_key_mask(shape, causal):
    """Per-batch key validity (prefix and holes); rows with at least one valid key
    match the masked baseline, rows with none come out non-finite as the baseline's."""
    b, h, s, hd = shape
    q, k, v = _qkv(shape, seed=31)
    g = torch.Generator().manual_seed(s)
    kv = torch.rand(b, s, generator=g) < 0.7
    kv[0, s // 2:] = False  # a prefix mask in batch 0
    out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal, key_valid=kv.to(DEV)).cpu()
    ref = _attention_ref_keymask(q, k, v, hd ** -0.5, causal, kv)
    allowed = torch.ones(s, s, dtype=torch.bool).tril() if causal else torch.ones(s, s, dtype=torch.bool)
    seen = (kv[:, None, :] & allowed[None]).any(-1)  # [b, s]: query rows with a valid key
    bad, err = or_rule_violations(out[seen], ref[seen])
    assert bad == 0, err
    assert not bool(torch.isfinite(out[~seen]).all()) or not bool((~seen).any())


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("pattern", ["tail", "head", "holes"])
def test_flash_attention_key_masked_loop_is_bit_identical(pattern, hd):
    """Causal with a key mask, head_dim 128 and 64: the generated key-masked loops
    (tk_attn_epochs_kmask.inc, tk_attn_steps64_kmask.inc) against the compiled
    epochs, forced as in
    test_flash_attention_epoch_loop_is_bit_identical by K/V rows 4 MiB apart.
    tail: padded keys at the end; head: the first 200 keys invalid, so query
    blocks enter the loop with rows that have seen no valid key (m = -inf);
    holes: about 30 % of keys invalid.  Rows with no valid key come out
    non-finite on both paths."""
    b, h, s = 2, 1, 1300
    q, k, v = _qkv((b, h, s, hd), seed=97)
    kv = torch.ones(b, s, dtype=torch.bool)
    if pattern == "tail":
        kv[0, 1000:] = False
        kv[1, 700:] = False
    elif pattern == "head":
        kv[:, :200] = False
    else:
        kv = torch.rand(b, s, generator=torch.Generator().manual_seed(5)) > 0.3
    qd, kd, vd, kvd = q.to(DEV), k.to(DEV), v.to(DEV), kv.to(DEV)
    compact = ops.flash_attention(qd, kd, vd, hd ** -0.5, True, key_valid=kvd)
    rs = 1 << 21
    wide_k = torch.zeros(b, s, rs, dtype=torch.float16, device=DEV)
    wide_v = torch.zeros(b, s, rs, dtype=torch.float16, device=DEV)
    wide_k[:, :, :hd] = kd[:, 0]
    wide_v[:, :, :hd] = vd[:, 0]
    kw, vw = wide_k[:, :, :hd][:, None], wide_v[:, :, :hd][:, None]
    assert kw.stride(2) == rs and torch.equal(kw, kd)
    spread = ops.flash_attention(qd, kw, vw, hd ** -0.5, True, key_valid=kvd)
    del wide_k, wide_v
    same = (compact == spread) | (torch.isnan(compact) & torch.isnan(spread))
    assert bool(same.all())
    ref = _attention_ref_keymask(q, k, v, hd ** -0.5, True, kv)
    seen = (kv[:, None, :] & torch.ones(s, s, dtype=torch.bool).tril()[None]).any(-1)
    bad, err = or_rule_violations(compact.cpu()[seen], ref[seen])
    assert bad == 0, err


def test_flash_attention_key_mask_256_row_blocks():
    """Causal head_dim 64 beyond 32768 keys runs 256-row query blocks (8 waves),
    whose key-masked steps come from tk_attn_steps64_w8_kmask.inc.  Padded tail
    (batch 0 from key 30000) and ~20 % random holes; sampled query rows (block
    edges, the padded tail, random rows) against the masked baseline softmax
    (src/torch_transformer_benchmark.py:97-112) over each row's full key range."""
    b, h, s, hd = 2, 2, 33000, 64
    q, k, v = _qkv((b, h, s, hd), seed=33)
    g = torch.Generator().manual_seed(7)
    kv = torch.rand(b, s, generator=g) > 0.2
    kv[0, 30000:] = False
    out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, True, key_valid=kv.to(DEV)).cpu()
    rows = torch.unique(torch.cat([torch.tensor([0, 1, 255, 256, 511, 16383, 32767, 32768, 29999, 30000, s - 2, s - 1]),
                                   torch.randint(0, s, (116,), generator=g)]))
    for bi in range(b):
        for hi in range(h):
            scores = torch.matmul(q[bi, hi, rows].float(), k[bi, hi].float().t()) * hd ** -0.5
            allowed = kv[bi][None, :] & (torch.arange(s)[None, :] <= rows[:, None])
            ref = torch.matmul(ob.masked_softmax_ref(scores, False, allowed), v[bi, hi].float())
            got = out[bi, rows, hi * hd:(hi + 1) * hd]
            seen = allowed.any(-1)
            bad, err = or_rule_violations(got[seen], ref[seen])
            assert bad == 0, (bi, hi, err)
            assert not bool(torch.isfinite(got[~seen]).any())


def test_attention_support_probes():
    """The reference's rule, next_pow2(max(hd, 16)) <= 256 for fp16 on the GPU
    (src/kernels.py:96-103); above it the kernel raises."""
    assert ops.attention_supported(64, torch.float16, DEV)
    assert ops.attention_supported(8, torch.float16, DEV)
    assert ops.attention_supported(100, torch.float16, DEV)
    assert ops.attention_supported(256, torch.float16, DEV)
    assert not ops.attention_supported(257, torch.float16, DEV)
    assert not ops.attention_supported(512, torch.float16, DEV)
    assert not ops.attention_supported(64, torch.float32, DEV)
    q = torch.zeros(1, 1, 8, 264, dtype=torch.float16, device=DEV)
    with pytest.raises(_lib.TkError, match="head_dim"):
        ops.flash_attention(q, q, q, 1.0, True)


# Head dims without a tile of their own (the element-load kernel on the next
# power-of-two tile), on and off the 64-key / 128-row grids.
ODD_HD_SHAPES = [(1, 2, 64, 1), (2, 3, 100, 24), (1, 2, 333, 40), (2, 2, 130, 100), (1, 2, 257, 200),
                 (1, 1, 70, 250)]


@pytest.mark.parametrize("shape", ODD_HD_SHAPES, ids=lambda s: "b{}h{}s{}d{}".format(*s))
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_flash_attention_any_head_dim(shape, causal):
    b, h, s, hd = shape
    q, k, v = _qkv(shape, seed=hd)
    out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal)
    assert out.shape == (b, s, h * hd)
    bad, err = or_rule_violations(out, ob.attention_ref(q, k, v, hd ** -0.5, causal))
    assert bad == 0, err


@pytest.mark.parametrize("hd", [24, 64, 128])
def test_flash_attention_unaligned_views(hd):
    """q/k/v views whose rows are not 16-byte vectors (a 3-element offset into
    one buffer, row stride not a multiple of 8) take the element-load path."""
    b, h, s = 2, 3, 150
    base = seeded(b * h * s * (hd + 3) + 3, dtype=torch.float16, seed=hd)
    ref_views = []
    dev_views = []
    for i in range(3):
        flat = base.roll(i * 17)
        t = flat[3:].view(b, h, s, hd + 3)[..., :hd]
        ref_views.append(t.contiguous())
        dev_views.append(flat.to(DEV)[3:].view(b, h, s, hd + 3)[..., :hd])
    for causal in (True, False):
        out = ops.flash_attention(*dev_views, hd ** -0.5, causal)
        bad, err = or_rule_violations(out, ob.attention_ref(*ref_views, hd ** -0.5, causal))
        assert bad == 0, (causal, err)


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
def test_flash_attention_any_head_dim_key_mask(causal):
    b, h, s, hd = 2, 2, 150, 48
    q, k, v = _qkv((b, h, s, hd), seed=48)
    g = torch.Generator().manual_seed(48)
    kv = torch.rand(b, s, generator=g) < 0.7
    kv[:, 0] = True
    out = ops.flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), hd ** -0.5, causal, key_valid=kv.to(DEV)).cpu()
    ref = _attention_ref_keymask(q, k, v, hd ** -0.5, causal, kv)
    bad, err = or_rule_violations(out, ref)
    assert bad == 0, err


# --------------------------------------------------------------------------- #
# Masked softmax
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("groups,s", [(3, 64), (2, 128), (4, 100), (2, 2048), (1, 5000)])
@pytest.mark.parametrize("causal", [True, False])
def test_masked_softmax(groups, s, causal):
    scores = seeded(groups, s, s, seed=s) * 3
    got = ops.masked_softmax(scores.to(DEV), causal)
    want = ob.masked_softmax_ref(scores, causal)
    assert (got.cpu().float() - want).abs().max() <= 1e-3  # fp16 cast of values in [0, 1]


def test_masked_softmax_key_lengths():
    b, h, s = 3, 2, 40
    scores = seeded(b * h, s, s, seed=77)
    key_len = torch.tensor([40, 17, 1], dtype=torch.int32)
    got = ops.masked_softmax(scores.to(DEV), True, key_len=key_len, heads_per_batch=h)
    valid = torch.arange(s)[None, :] < key_len[:, None]  # [B, S]
    want = torch.stack([ob.masked_softmax_ref(scores[g], True, valid[g // h]) for g in range(b * h)])
    want = torch.nan_to_num(want, nan=0.0)  # all-masked rows -> zeros
    assert (got.cpu().float() - want).abs().max() <= 1e-3


def test_gelu_epilogue_dense_range():
    """The GELU epilogue over a dense sweep of pre-activations: A = 0 so the
    GEMM output is gelu(bias) exactly; compared with the exact-erf GELU cast
    to fp16.  The kernel's formula (max(x, 0) - |x|*2^P(|x|), P a fitted
    degree-5 polynomial) carries |GELU error| <= 7.2e-7 on [-12, 12]
    (tests/test_gelu_poly.py); where |GELU| ~ 1e-3 one fp16 ulp is ~1e-6, so
    the allowed difference is max(1 ulp, 2e-6)."""
    n = 8192
    bias = torch.linspace(-8.0, 8.0, n)
    a = torch.zeros(64, 64, dtype=torch.float16, device=DEV)
    w = torch.zeros(n, 64, dtype=torch.float16, device=DEV)
    got = ops.linear(a, w, bias.to(DEV), gelu=True)
    want = ob.gelu_ref(bias).half().float().expand(64, n)
    assert fp16_excess(got, want, atol=2e-6) <= 0
