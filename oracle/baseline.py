"""fp32 CPU restatement of the reference transformer and its harness helpers.

TEST INFRASTRUCTURE ONLY -- the product never imports this module.

Every function cites the reference code it restates (paths relative to the
reference repository).  The module tree is built in the same order as the
reference so that ``torch.manual_seed(s)`` followed by construction consumes
the RNG identically and yields bit-identical weights and ``state_dict`` keys.

Pinning (see tests/test_oracle.py):
  * ``BaselineTransformer`` construction and ``forward``: golden vectors written
    by ``tests/golden/make_golden.py`` from the reference itself (seeded weight
    hashes and outputs, bit-exact), plus the float64 twin in ``twin64``.
  * ``layer_norm_ref`` / ``add_layer_norm_ref``: ``F.layer_norm`` and the
    closed-form population-variance LayerNorm in float64.
  * ``gelu_ref``: closed form 0.5*x*(1+erf(x/sqrt 2)) from ``math.erf``.
  * ``attention_ref`` / ``masked_softmax_ref``: brute-force float64 loops on
    tiny shapes, softmax row sums == 1, causal rows ignore future keys.
  * ``compare_outputs``: hand-built cases for every branch of the OR rule
    (NaN/inf fail, relative term uses |ref|).
  * ``chunked_forward`` / ``sampled_rows_forward``: equal to the unchunked
    ``BaselineTransformer`` at feasible sizes (the chain-of-trust method of
    src/run_case14.py:165-221).
"""

from __future__ import annotations

import math
import statistics
import time
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

ATOL = 0.002  # src/torch_transformer_benchmark.py:619 (argparse default)
RTOL = 0.02  # src/torch_transformer_benchmark.py:618


# --------------------------------------------------------------------------- #
# Config (src/torch_transformer_benchmark.py:29-56)
# --------------------------------------------------------------------------- #


@dataclass(frozen=True)
class TransformerConfig:
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
                f"d_model ({self.d_model}) must be divisible by "
                f"num_heads ({self.num_heads})"
            )
        if self.ffn_dim <= 0:
            raise ValueError("ffn_dim must be positive")
        if self.num_layers <= 0:
            raise ValueError("num_layers must be positive")


# --------------------------------------------------------------------------- #
# Model (src/torch_transformer_benchmark.py:59-172)
# --------------------------------------------------------------------------- #


class BaselineSelfAttention(nn.Module):
    """Restates src/torch_transformer_benchmark.py:59-122.

    Construction order q, k, v, out (:72-75) fixes RNG consumption.
    """

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

    def _heads(self, t: torch.Tensor) -> torch.Tensor:
        # [B, S, D] -> [B, H, S, hd] contiguous (:77-83)
        b, s, _ = t.shape
        return t.view(b, s, self.num_heads, self.head_dim).transpose(1, 2).contiguous()

    def forward(self, x, valid_token_mask=None, causal=False):
        b, s, _ = x.shape
        q = self._heads(self.q_proj(x))
        k = self._heads(self.k_proj(x))
        v = self._heads(self.v_proj(x))
        # scale applied after the matmul, in the activation dtype (:97)
        scores = torch.matmul(q, k.transpose(-2, -1)) * self.scale
        if causal:  # (:99-103)
            future = torch.ones((s, s), device=x.device, dtype=torch.bool).triu(1)
            scores = scores.masked_fill(future, float("-inf"))
        if valid_token_mask is not None:  # key mask (:105-108)
            scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(dtype=x.dtype)  # (:111)
        ctx = torch.matmul(probs, v)
        ctx = ctx.transpose(1, 2).contiguous().view(b, s, self.d_model)  # (:113-117)
        out = self.out_proj(ctx)
        if valid_token_mask is not None:  # (:120-121)
            out = out.masked_fill(~valid_token_mask[..., None], 0)
        return out


class BaselineTransformerBlock(nn.Module):
    """Restates src/torch_transformer_benchmark.py:125-145 (pre-LN block).

    Construction order norm1, attention, norm2, ffn_in, ffn_out (:128-132).
    """

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = BaselineSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x, valid_token_mask, causal):
        x = x + self.attention(self.norm1(x), valid_token_mask, causal)
        x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class BaselineTransformer(nn.Module):
    """Restates src/torch_transformer_benchmark.py:148-172 (layers, final LN)."""

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

    def forward(self, x, valid_token_mask=None):
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal)
        x = self.final_norm(x)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


def copy_model_weights(baseline: nn.Module, optimized: nn.Module, strict: bool = True):
    """Strict state_dict copy (src/torch_transformer_benchmark.py:203-213)."""
    state = {k: v.detach().clone() for k, v in baseline.state_dict().items()}
    return optimized.load_state_dict(state, strict=strict)


def build_model(config, seed: int = 1234) -> BaselineTransformer:
    """Seeded construction as the harness does it (:683,690)."""
    torch.manual_seed(seed)
    return BaselineTransformer(config)


# --------------------------------------------------------------------------- #
# Inputs (src/torch_transformer_benchmark.py:234-272)
# --------------------------------------------------------------------------- #


def generate_random_case(
    config,
    device="cpu",
    dtype=torch.float32,
    seed: int = 1234,
    padding_ratio: float = 0.0,
    input_scale: float = 1.0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Seeded input and valid-token mask.

    Generated with a generator on ``device`` exactly as the harness does; the
    build's tests call it with device="cpu" and copy to the GPU, because CPU
    and GPU generators produce different streams.
    """
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    x = torch.randn(
        config.batch_size, config.seq_len, config.d_model,
        generator=gen, device=device, dtype=dtype,
    )
    x = x * input_scale
    if padding_ratio <= 0:
        mask = torch.ones(config.batch_size, config.seq_len, device=device, dtype=torch.bool)
        return x, mask
    min_valid = max(1, int(round(config.seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(
        low=min_valid, high=config.seq_len + 1, size=(config.batch_size,),
        generator=gen, device=device,
    )
    mask = torch.arange(config.seq_len, device=device)[None, :] < lengths[:, None]
    x = x.masked_fill(~mask[..., None], 0)
    return x, mask


# --------------------------------------------------------------------------- #
# Accuracy rule (src/torch_transformer_benchmark.py:275-356)
# --------------------------------------------------------------------------- #


@dataclass
class AccuracyResult:
    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float


def compare_outputs(reference, optimized, rtol: float = RTOL, atol: float = ATOL) -> AccuracyResult:
    """Exact OR rule: |d| <= atol OR |d| <= rtol*|ref|; non-finite fails."""
    if reference.shape != optimized.shape:
        raise AssertionError(
            f"shape mismatch: baseline={tuple(reference.shape)}, "
            f"optimized={tuple(optimized.shape)}"
        )
    ref = reference.detach().float().cpu()
    opt = optimized.detach().float().cpu()
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    err = (opt - ref).abs()
    ok = finite & ((err <= atol) | (err <= rtol * ref.abs()))
    failed = ~ok
    n_failed = int(failed.sum().item())
    flat = int(err.reshape(-1).argmax().item()) if err.numel() else 0
    worst = tuple(int(i) for i in torch.unravel_index(torch.tensor(flat), ref.shape)) if ref.ndim else ()
    rel = err / ref.abs().clamp_min(1e-12)
    if ref.ndim == 0:
        dims = [0] if n_failed else []
    elif ref.ndim == 1:
        dims = torch.nonzero(failed).flatten().tolist()
    else:
        dims = torch.nonzero(failed.any(dim=tuple(range(ref.ndim - 1)))).flatten().tolist()
    return AccuracyResult(
        passed=n_failed == 0,
        total_elements=ref.numel(),
        failed_elements=n_failed,
        max_abs_error=float(err.max().item()) if err.numel() else 0.0,
        max_relative_error=float(rel.max().item()) if rel.numel() else 0.0,
        mean_abs_error=float(err.mean().item()) if err.numel() else 0.0,
        failed_feature_dims=dims,
        worst_index=worst,
        reference_at_worst=float(ref[worst].item()) if ref.numel() else 0.0,
        optimized_at_worst=float(opt[worst].item()) if opt.numel() else 0.0,
    )


# --------------------------------------------------------------------------- #
# Per-kernel references
# --------------------------------------------------------------------------- #


def layer_norm_ref(x, weight, bias, eps=1e-5, out_dtype=None):
    """fp32 LayerNorm then cast (src/fused_kernels.py:80-112 numerics)."""
    y = F.layer_norm(x.float(), (x.shape[-1],), weight.float(), bias.float(), eps)
    return y if out_dtype is None else y.to(out_dtype)


def add_layer_norm_ref(x, y, weight, bias, eps=1e-5, out_dtype=None):
    """s = x + y in fp32; h = LN(s) cast (src/fused_kernels.py:114-161)."""
    s = x.float() + y.float()
    return s, layer_norm_ref(s, weight, bias, eps, out_dtype)


def gelu_ref(x):
    """Exact (erf) GELU as F.gelu(approximate='none') (src/torch_transformer_benchmark.py:141)."""
    return F.gelu(x.float(), approximate="none")


def masked_softmax_ref(scores, causal: bool, key_valid: Optional[torch.Tensor] = None):
    """fp32 softmax over the last dim after -inf masking.

    Baseline order (src/torch_transformer_benchmark.py:99-111,
    src/optimized.py:658-666): causal triu(1) -> key mask -> softmax(fp32).
    ``scores``: [..., Sq, Sk] with query i aligned to key i.
    """
    s = scores.float()
    sq, sk = s.shape[-2], s.shape[-1]
    if causal:
        future = torch.ones((sq, sk), dtype=torch.bool).triu(1)
        s = s.masked_fill(future, float("-inf"))
    if key_valid is not None:
        s = s.masked_fill(~key_valid, float("-inf"))
    return torch.softmax(s, dim=-1)


def attention_ref(q, k, v, scale: float, causal: bool):
    """Reference attention in the baseline op order, fp32 throughout.

    q/k/v: [B, H, S, hd] (any float dtype; promoted to fp32).  Returns the
    context as [B, S, H*hd] fp32 (src/test_triton_kernels.py:125-139 order:
    fp32 scores -> post-scale -> -inf triu mask -> softmax -> PV).
    """
    qf, kf, vf = q.float(), k.float(), v.float()
    scores = torch.matmul(qf, kf.transpose(-2, -1)) * scale
    probs = masked_softmax_ref(scores, causal)
    ctx = torch.matmul(probs, vf)
    b, h, s, hd = ctx.shape
    return ctx.transpose(1, 2).reshape(b, s, h * hd)


# --------------------------------------------------------------------------- #
# Long-sequence references (chain of trust of src/run_case14.py:165-221)
# --------------------------------------------------------------------------- #


def _attention_rows(layer, h, rows: Optional[torch.Tensor], causal: bool, q_chunk: int):
    """Attention output (pre-residual) for query rows ``rows`` (all if None).

    Keys/values are projected for every token; queries only for ``rows``.
    Each query chunk forms its own [B, H, chunk, S] score block, so the peak
    memory is bounded while every row's arithmetic is the baseline's.
    """
    attn = layer.attention
    b, s, d = h.shape
    nh, hd = attn.num_heads, attn.head_dim
    k = attn._heads(attn.k_proj(h))
    v = attn._heads(attn.v_proj(h))
    row_idx = torch.arange(s) if rows is None else rows
    out = torch.empty(b, row_idx.numel(), d, dtype=h.dtype)
    for c0 in range(0, row_idx.numel(), q_chunk):
        idx = row_idx[c0 : c0 + q_chunk]
        q = attn.q_proj(h[:, idx, :]).view(b, idx.numel(), nh, hd).transpose(1, 2).contiguous()
        # Causal: keys past the chunk's last query are -inf for every row of
        # the chunk, i.e. contribute exactly 0; they are left out.
        nk = int(idx.max()) + 1 if causal else s
        kc, vc = k[:, :, :nk, :], v[:, :, :nk, :]
        scores = torch.matmul(q, kc.transpose(-2, -1)) * attn.scale
        if causal:
            future = torch.arange(nk)[None, :] > idx[:, None]
            scores = scores.masked_fill(future, float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(h.dtype)
        ctx = torch.matmul(probs, vc).transpose(1, 2).contiguous().view(b, idx.numel(), d)
        out[:, c0 : c0 + idx.numel(), :] = attn.out_proj(ctx)
    return out


@torch.no_grad()
def chunked_forward(model: BaselineTransformer, x: torch.Tensor, q_chunk: int = 1024):
    """Dense-mask forward, attention chunked over query rows.

    Row-exact restatement of ``BaselineTransformer.forward`` without the
    [B, H, S, S] score tensor, for shapes whose full score tensor does not fit
    host memory (configs with S >= 8192).
    """
    causal = model.config.causal
    for layer in model.layers:
        x = x + _attention_rows(layer, layer.norm1(x), None, causal, q_chunk)
        x = x + layer.ffn_out(F.gelu(layer.ffn_in(layer.norm2(x)), approximate="none"))
    return model.final_norm(x)


@torch.no_grad()
def sampled_rows_forward(
    model: BaselineTransformer, x: torch.Tensor, rows: torch.Tensor, q_chunk: int = 512
):
    """Model output at query rows ``rows`` only, for a ONE-layer model.

    With one layer, output row i depends on x[:, :i+1] (causal) or on all of
    x (full) only through K/V of layer 0, which are computed for every token;
    everything after attention is row-local.  Returns [B, len(rows), D].
    """
    if len(model.layers) != 1:
        raise ValueError("sampled_rows_forward is exact only for one layer")
    layer = model.layers[0]
    a = _attention_rows(layer, layer.norm1(x), rows, model.config.causal, q_chunk)
    xr = x[:, rows, :] + a
    xr = xr + layer.ffn_out(F.gelu(layer.ffn_in(layer.norm2(xr)), approximate="none"))
    return model.final_norm(xr)


def sample_query_rows(seq_len: int, count: int = 512, seed: int = 1234) -> torch.Tensor:
    """The C5 check rows: CPU generator seeded ``seed``, randperm(S)[:count], sorted."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randperm(seq_len, generator=gen)[:count].sort().values


# --------------------------------------------------------------------------- #
# CPU timing (src/torch_transformer_benchmark.py:501-506, median as :564)
# --------------------------------------------------------------------------- #


def time_cpu_forward(model, x, warmup: int = 1, repeats: int = 3, fn=None) -> List[float]:
    """perf_counter_ns samples (ms) of ``fn(x)`` (default ``model(x)``)."""
    call = fn if fn is not None else model
    samples = []
    with torch.inference_mode():
        for _ in range(warmup):
            call(x)
        for _ in range(repeats):
            t0 = time.perf_counter_ns()
            call(x)
            samples.append((time.perf_counter_ns() - t0) / 1e6)
    return samples


def median(values: Sequence[float]) -> float:
    return statistics.median(values)


def gemm_flops(config) -> float:
    """2T(4D^2 + 2DF) per layer times L."""
    t = config.batch_size * config.seq_len
    d, f = config.d_model, config.ffn_dim
    return 2.0 * t * (4 * d * d + 2 * d * f) * config.num_layers


def attention_flops(config) -> float:
    """4*B*H*hd*P per layer, P = S(S+1)/2 causal, S^2 full."""
    s = config.seq_len
    pairs = s * (s + 1) / 2 if config.causal else s * s
    return 4.0 * config.batch_size * config.d_model * pairs * config.num_layers
