"""Tensor-level wrappers over libtkmi's kernels (device tensors in, device tensors out).

Names and argument meanings follow the reference's kernel wrappers:
  ``can_fuse``, ``ln_fwd``, ``add_ln_fwd``      -- src/fused_kernels.py:62-64,164-238
  ``attention_supported``, ``flash_attention``  -- src/kernels.py:96-103,250-294
plus the GEMM entry points that replace ``F.linear`` (+GELU / +residual /
+residual+LayerNorm) and the standalone masked softmax.

Every wrapper launches on torch's current HIP stream and allocates its
outputs with ``torch.empty`` (the caching allocator).  There is no CPU or
torch fallback: a CPU tensor, an unsupported dtype or a missing library
raises.
"""

from __future__ import annotations

import contextlib
from typing import List, Optional, Tuple

import torch

from . import _lib
from ._lib import (TK_EPI_BIAS, TK_EPI_BIAS_GELU, TK_EPI_BIAS_RESID, TK_F16, TK_F32, TK_ROWS_KEEP_RESID,
                   TK_ROWS_ZERO, TK_ROWS_ZERO_ALL)

MAX_FUSED_SIZE = 8192  # longest LayerNorm row (src/fused_kernels.py:59)

_DTYPE_CODE = {torch.float32: TK_F32, torch.float16: TK_F16}


# --------------------------------------------------------------------------- #
# Per-kernel timing (used by bench.py): events recorded on the launch stream.
# --------------------------------------------------------------------------- #

_timer: Optional[List[Tuple[str, "torch.cuda.Event", "torch.cuda.Event"]]] = None


@contextlib.contextmanager
def kernel_timer():
    """Collect (name, start_event, end_event) around every kernel launched inside."""
    global _timer
    prev, _timer = _timer, []
    try:
        yield _timer
    finally:
        _timer = prev


def _launch(name: str, fn: str, *args) -> None:
    if _timer is None:
        _lib.call(fn, *args)
        return
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    _lib.call(fn, *args)
    end.record()
    _timer.append((name, start, end))


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "tkmi kernels run on the GPU only; got a tensor on "
                f"{t.device} (there is no CPU path)"
            )


def _code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32 or float16") from None


# --------------------------------------------------------------------------- #
# LayerNorm (src/fused_kernels.py:164-238)
# --------------------------------------------------------------------------- #


def can_fuse(x: torch.Tensor) -> bool:
    """Whether the LayerNorm kernels take rows shaped like ``x``."""
    return x.is_cuda and x.shape[-1] <= MAX_FUSED_SIZE and _lib.is_available()


def _row_mask(mask, rows: int):
    """A [rows] byte view of a bool / uint8 validity mask (nonzero = valid), or None."""
    if mask is None:
        return None
    if mask.numel() != rows or mask.dtype not in (torch.bool, torch.uint8):
        raise ValueError(f"row mask must be bool/uint8 with {rows} elements, got {mask.dtype} {tuple(mask.shape)}")
    _require_cuda(mask)
    return mask.reshape(rows).contiguous()


def ln_fwd(x, weight, bias, eps: float, out_dtype: Optional[torch.dtype] = None, out=None,
           name: str = "ln_cast", row_valid=None):
    """LayerNorm over the last dim, fp32 statistics, output in ``out_dtype``.

    ``row_valid`` (optional bool mask over the rows): invalid rows are written
    as zeros (the masked final norm, src/torch_transformer_benchmark.py:170-171).
    """
    _require_cuda(x, weight, bias)
    out_dtype = x.dtype if out_dtype is None else out_dtype
    shape = x.shape
    cols = shape[-1]
    x2 = x.float().contiguous().view(-1, cols)
    w = weight.float().contiguous()
    b = bias.float().contiguous()
    if out is None:
        out = torch.empty(x2.shape, dtype=out_dtype, device=x.device)
    rv = _row_mask(row_valid, x2.shape[0])
    _launch(
        name, "tk_ln_cast", x2.data_ptr(), w.data_ptr(), b.data_ptr(), out.data_ptr(),
        _code(out_dtype), x2.shape[0], cols, float(eps), rv.data_ptr() if rv is not None else None, _stream(x),
    )
    return out.view(shape)


def add_ln_fwd(x, y, weight, bias, eps: float, out_dtype: Optional[torch.dtype] = None,
               write_sum: bool = True):
    """Residual add + LayerNorm: returns ``(s, h)``, h = LN(s).

    As src/fused_kernels.py:196-238: ``s = x + y`` is added in fp32 and
    returned in ``x``'s dtype (float32 or float16); the statistics use the
    fp32 sum; ``h`` is in ``out_dtype`` (default ``x.dtype``).  With
    ``write_sum=False`` the sum is not stored and ``s`` is None (the final
    norm of the model, src/optimized.py:542-553).
    """
    _require_cuda(x, y, weight, bias)
    if x.shape != y.shape:
        raise ValueError(f"shape mismatch: {tuple(x.shape)} vs {tuple(y.shape)}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    shape = x.shape
    cols = shape[-1]
    x2 = x.contiguous().view(-1, cols)
    y2 = y.contiguous().view(-1, cols)
    w = weight.float().contiguous()
    b = bias.float().contiguous()
    s = torch.empty_like(x2) if write_sum else None
    h = torch.empty(x2.shape, dtype=out_dtype, device=x.device)
    _launch(
        "add_ln_cast", "tk_add_ln_cast", x2.data_ptr(), _code(x2.dtype), y2.data_ptr(), _code(y2.dtype),
        w.data_ptr(), b.data_ptr(), s.data_ptr() if s is not None else None, h.data_ptr(),
        _code(out_dtype), x2.shape[0], cols, float(eps), _stream(x),
    )
    return (s.view(shape) if s is not None else None), h.view(shape)


# --------------------------------------------------------------------------- #
# GEMMs (replace F.linear, src/optimized.py:572,627,632-636)
# --------------------------------------------------------------------------- #


def _check_gemm_operands(a: torch.Tensor, w: torch.Tensor):
    _require_cuda(a, w)
    if a.dtype != torch.float16 or w.dtype != torch.float16:
        raise TypeError(f"GEMM operands must be float16, got {a.dtype} and {w.dtype}")
    if a.dim() != 2 or w.dim() != 2 or a.shape[1] != w.shape[1]:
        raise ValueError(f"GEMM shapes {tuple(a.shape)} x {tuple(w.shape)}^T do not match")
    if a.stride(1) != 1 or w.stride(1) != 1:
        raise ValueError("GEMM operands must be K-contiguous")


def linear(a, w, bias=None, gelu: bool = False, out=None, name: Optional[str] = None):
    """fp16 ``[M, N] = a[M, K] . w[N, K]^T + bias`` (optionally exact GELU), fp32 accumulate."""
    _check_gemm_operands(a, w)
    m, k = a.shape
    n = w.shape[0]
    if out is None:
        out = torch.empty((m, n), dtype=torch.float16, device=a.device)
    _launch(
        name or ("gemm_gelu" if gelu else "gemm"), "tk_gemm", a.data_ptr(), a.stride(0), w.data_ptr(),
        w.stride(0), bias.data_ptr() if bias is not None else None, None, 0, out.data_ptr(),
        out.stride(0), m, n, k, TK_EPI_BIAS_GELU if gelu else TK_EPI_BIAS, None, 0, _stream(a),
    )
    return out


def linear_residual(a, w, bias, resid, out=None, name: str = "gemm_resid", row_valid=None,
                    row_mode: int = TK_ROWS_KEEP_RESID):
    """fp32 ``out = resid + a . w^T + bias``; ``out`` may be ``resid`` (in place).

    ``row_valid`` (optional bool mask over the M rows): an invalid row becomes
    ``resid`` (``TK_ROWS_KEEP_RESID``) or 0 (``TK_ROWS_ZERO``).
    """
    _check_gemm_operands(a, w)
    m, k = a.shape
    n = w.shape[0]
    if resid.dtype != torch.float32 or tuple(resid.shape) != (m, n) or resid.stride(1) != 1:
        raise ValueError("residual must be fp32 [M, N] with contiguous rows")
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    rv = _row_mask(row_valid, m)
    _launch(
        name, "tk_gemm", a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0),
        bias.data_ptr() if bias is not None else None, resid.data_ptr(), resid.stride(0),
        out.data_ptr(), out.stride(0), m, n, k, TK_EPI_BIAS_RESID, rv.data_ptr() if rv is not None else None,
        int(row_mode) if rv is not None else 0, _stream(a),
    )
    return out


def gemm_ln_supported(n: int) -> bool:
    return bool(_lib.load().tk_gemm_ln_supported(int(n)))


def linear_add_ln(a, w, bias, resid, ln_weight, ln_bias, eps: float, out_dtype=torch.float16,
                  sum_out=None, h_out=None, name: str = "gemm_add_ln", row_valid=None,
                  row_mode: int = TK_ROWS_KEEP_RESID):
    """``s = resid + a . w^T + bias``; ``h = LN(s)`` in one kernel (full-row tiles).

    ``sum_out`` receives s when given (it may be ``resid``); returns h.
    ``row_valid`` / ``row_mode``: an invalid row takes s = resid
    (``TK_ROWS_KEEP_RESID``) or s = 0 (``TK_ROWS_ZERO``; ``TK_ROWS_ZERO_ALL``
    also writes h = 0).
    """
    _check_gemm_operands(a, w)
    m, k = a.shape
    n = w.shape[0]
    if resid.dtype != torch.float32 or not resid.is_contiguous() or tuple(resid.shape) != (m, n):
        raise ValueError("residual must be contiguous fp32 [M, N]")
    if h_out is None:
        h_out = torch.empty((m, n), dtype=out_dtype, device=a.device)
    rv = _row_mask(row_valid, m)
    _launch(
        name, "tk_gemm_bias_add_ln", a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0),
        bias.data_ptr() if bias is not None else None, resid.data_ptr(), ln_weight.data_ptr(),
        ln_bias.data_ptr(), sum_out.data_ptr() if sum_out is not None else None, h_out.data_ptr(),
        _code(h_out.dtype), m, n, k, float(eps), rv.data_ptr() if rv is not None else None,
        int(row_mode) if rv is not None else 0, _stream(a),
    )
    return h_out


# --------------------------------------------------------------------------- #
# Attention (src/kernels.py:96-103,250-294)
# --------------------------------------------------------------------------- #


def attention_supported(head_dim: int, dtype: torch.dtype = torch.float16, device=None) -> bool:
    """Whether ``flash_attention`` handles this head_dim / dtype / device."""
    if device is not None and torch.device(device).type != "cuda":
        return False
    if dtype != torch.float16:
        return False
    return bool(_lib.load().tk_attention_supported(int(head_dim)))


def flash_attention(q, k, v, scale: float, causal: bool, out=None, key_valid=None):
    """Exact attention; returns the context as ``[B, S, H*hd]`` fp16.

    q/k/v are logically ``[B, H, S, hd]`` fp16 and may be strided views in
    the first three dims (e.g. of the fused ``[B, S, 3, H, hd]`` projection);
    the last dim must be contiguous.  ``key_valid`` (optional ``[B, S]`` bool):
    invalid keys are masked like future keys
    (src/torch_transformer_benchmark.py:105-108); a query row with no valid
    key comes out non-finite, as the baseline's.
    """
    _require_cuda(q, k, v)
    bsz, nh, s, hd = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must share one shape")
    if q.dtype != torch.float16 or k.dtype != torch.float16 or v.dtype != torch.float16:
        raise TypeError("flash_attention takes float16 q/k/v")
    if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("flash_attention needs a contiguous head_dim")
    if out is None:
        out = torch.empty((bsz, s, nh * hd), dtype=torch.float16, device=q.device)
    o_strides = (out.stride(0), hd, out.stride(1))
    kv = None
    if key_valid is not None:
        if tuple(key_valid.shape) != (bsz, s):
            raise ValueError(f"key_valid must be [B, S] = {(bsz, s)}, got {tuple(key_valid.shape)}")
        kv = _row_mask(key_valid, bsz * s)
    _launch(
        "flash_attn", "tk_flash_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        bsz, nh, s, hd, _lib.strides3(q.stride()[:3]), _lib.strides3(k.stride()[:3]),
        _lib.strides3(v.stride()[:3]), _lib.strides3(o_strides), float(scale), int(bool(causal)),
        kv.data_ptr() if kv is not None else None, s, _stream(q),
    )
    return out


def qkv_attention_supported(batch: int, seq: int, heads: int, head_dim: int) -> bool:
    return bool(_lib.load().tk_qkv_attention_supported(batch, seq, heads, head_dim))


def qkv_attention(h, w_qkv, b_qkv, batch: int, seq: int, heads: int, head_dim: int, scale: float,
                  causal: bool, out=None, name: str = "qkv_attn"):
    """Fused ``F.linear(h, w_qkv, b_qkv)`` + attention for one-key-tile sequences.

    ``h`` [batch*seq, d] fp16, ``w_qkv`` [3d, d] fp16 (q, k, v rows), ``b_qkv``
    [3d] fp32; returns the context ``[batch*seq, d]`` fp16 -- what
    ``linear`` into a q|k|v buffer followed by ``flash_attention`` on its
    views gives (src/optimized.py:572-626), without the q|k|v buffer.
    """
    _require_cuda(h, w_qkv, b_qkv)
    _check_gemm_operands(h, w_qkv)
    d = heads * head_dim
    if tuple(h.shape) != (batch * seq, d) or tuple(w_qkv.shape) != (3 * d, d) or tuple(b_qkv.shape) != (3 * d,):
        raise ValueError("qkv_attention: h [B*S, d], w_qkv [3d, d], b_qkv [3d] expected")
    if b_qkv.dtype != torch.float32 or not b_qkv.is_contiguous():
        raise TypeError("qkv_attention: b_qkv must be contiguous fp32")
    if out is None:
        out = torch.empty((batch * seq, d), dtype=torch.float16, device=h.device)
    _launch(
        name, "tk_qkv_attention", h.data_ptr(), h.stride(0), w_qkv.data_ptr(), w_qkv.stride(0), b_qkv.data_ptr(),
        out.data_ptr(), out.stride(0), batch, seq, heads, head_dim, float(scale), int(bool(causal)), _stream(h),
    )
    return out


def small_forward_supported(seq: int, d_model: int, heads: int, head_dim_padded: int, ffn_dim: int) -> bool:
    return bool(_lib.load().tk_small_forward_supported(seq, d_model, heads, head_dim_padded, ffn_dim))


def small_forward(x, out, stacked: dict, final: tuple, n1_eps: float, n2_eps: float, heads: int,
                  head_dim_padded: int, ffn_dim: int, causal: bool, scale: float, name: str = "small_forward"):
    """The whole dense forward of a narrow model in one launch (tk_small_forward).

    x, out: [B, S, D] fp32 contiguous; ``stacked``: the layers' packed weights
    stacked over layers (OptimizedTransformer._stacked_weights); ``final`` =
    (weight, bias, eps) of the final LayerNorm.
    """
    _require_cuda(x, out)
    if x.dtype != torch.float32 or out.dtype != torch.float32 or not x.is_contiguous() or not out.is_contiguous():
        raise ValueError("small_forward: x and out must be contiguous fp32")
    b, s, d = x.shape
    w = stacked
    layers = w["w_qkv"].shape[0]
    nf_w, nf_b, nf_eps = final
    _launch(name, "tk_small_forward", x.data_ptr(), out.data_ptr(), b, s, d, heads, head_dim_padded, ffn_dim,
            layers, int(causal), w["w_qkv"].data_ptr(), w["b_qkv"].data_ptr(), w["w_o"].data_ptr(),
            w["b_o"].data_ptr(), w["w_1"].data_ptr(), w["b_1"].data_ptr(), w["w_2"].data_ptr(),
            w["b_2"].data_ptr(), w["n1_w"].data_ptr(), w["n1_b"].data_ptr(), w["n2_w"].data_ptr(),
            w["n2_b"].data_ptr(), nf_w.data_ptr(), nf_b.data_ptr(), float(n1_eps), float(n2_eps),
            float(nf_eps), float(scale), _stream(x))
    return out


def masked_softmax(scores, causal: bool, key_len=None, heads_per_batch: int = 1):
    """fp16 softmax of fp32 ``scores [..., S, S]`` with causal / per-batch key-length masking.

    ``key_len`` (optional, one int per batch): the kernel reads the length of
    score group g at ``key_len[g // heads_per_batch]``, so the groups must be
    whole batches of ``heads_per_batch`` heads and ``key_len`` must hold one
    entry per batch.
    """
    if scores.dtype != torch.float32 or scores.dim() < 2 or scores.shape[-1] != scores.shape[-2]:
        raise ValueError("scores must be fp32 [..., S, S]")
    s = scores.shape[-1]
    groups = scores.numel() // (s * s) if s else 0
    if key_len is not None:
        hpb = int(heads_per_batch)
        if hpb < 1 or groups % hpb != 0 or key_len.numel() * hpb != groups:
            raise ValueError(f"key_len needs one entry per batch of {heads_per_batch} heads: {groups} score groups, "
                             f"{key_len.numel()} lengths")
    _require_cuda(scores)
    sc = scores.contiguous()
    probs = torch.empty(sc.shape, dtype=torch.float16, device=sc.device)
    kl = None
    if key_len is not None:
        kl = key_len.to(device=sc.device, dtype=torch.int32).contiguous()
    _launch(
        "masked_softmax", "tk_masked_softmax", sc.data_ptr(), probs.data_ptr(), groups, s,
        int(bool(causal)), kl.data_ptr() if kl is not None else None, int(heads_per_batch),
        _stream(sc),
    )
    return probs
