"""The whole-forward kernel for narrow models (tk_small_forward).

Checked on the shapes it takes (S <= 128, d_model = ffn_dim = 128, attention
width 128 with head_dim 16/32/64/128, causal and not) against
  * the CPU oracle, with the harness's rule |d| <= 0.002 or |d| <= 0.02|ref|
    (src/torch_transformer_benchmark.py:309-316);
  * the layer-by-layer HIP path on the same weights and input (same
    arithmetic, different fp16 rounding points -- LayerNorm sums, and P
    rounded per 32-key block here against the layer path's key tiles):
    within 1e-3 of each other (measured at most 6.3e-4 over these shapes),
    and the whole-forward kernel's worst error against the oracle no more
    than 1e-4 above the layer path's (measured at most 2e-5 above).
A padded input, and a shape outside the envelope, take the layer path.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from oracle import baseline as ob

import tkmi

pytestmark = pytest.mark.gpu
DEV = "cuda"

SHAPES = [
    (64, 128, 128, 4, 128, 4, True),   # reference config 1
    (3, 32, 128, 4, 128, 2, True),     # appendix case 12's sequence length
    (3, 77, 128, 2, 128, 3, False),    # ragged S, non-causal, head_dim 64
    (4, 128, 128, 1, 128, 2, True),    # head_dim 128
    (2, 100, 128, 8, 128, 2, True),    # head_dim 16
    (2, 128, 128, 4, 128, 1, False),
    (1, 1, 128, 4, 128, 2, True),      # one token
    (2, 50, 128, 4, 128, 2, True),     # two row blocks: waves 4-7 own one valid block
    (3, 64, 128, 2, 128, 2, False),
    (2, 96, 128, 1, 128, 1, True),     # three row blocks, head_dim 128
]


def _pair(shape, seed=1234):
    cfg = ob.TransformerConfig(*shape)
    base = ob.build_model(cfg, seed=seed).eval()
    opt = tkmi.OptimizedTransformer(tkmi.TransformerConfig(*shape))
    ob.copy_model_weights(base, opt, strict=True)
    return base, opt.to(DEV).eval()


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "b{}_s{}_h{}_l{}_{}".format(s[0], s[1], s[3], s[5], "c" if s[6] else "nc"))
def test_small_forward_parity(shape):
    base, opt = _pair(shape)
    b, s, d = shape[0], shape[1], shape[2]
    assert opt._small_forward_ok(s, opt._weights())
    x = torch.randn(b, s, d, generator=torch.Generator().manual_seed(7 + s))
    with torch.inference_mode():
        got = opt(x.to(DEV))
        opt.settings = replace(opt.settings, small_forward=False)
        layered = opt(x.to(DEV))
    with torch.no_grad():
        ref = base(x)
    res = ob.compare_outputs(ref, got.cpu())
    res_layered = ob.compare_outputs(ref, layered.cpu())
    between = (got - layered).abs().max().item()
    print(f"{shape}: max_abs={res.max_abs_error:.3g} layered={res_layered.max_abs_error:.3g} "
          f"between={between:.3g} failed={res.failed_elements}", flush=True)
    assert res.passed, (res.max_abs_error, res.failed_elements)
    assert torch.isfinite(got).all()
    assert between <= 1e-3
    assert res.max_abs_error <= res_layered.max_abs_error + 1e-4


def test_small_forward_is_deterministic_and_batch_independent():
    """A sequence's rows are computed the same way whatever else the batch
    holds: a batch's outputs equal the outputs of its sequences run alone,
    bit for bit, and reruns are identical."""
    _, opt = _pair((4, 96, 128, 4, 128, 2, True))
    x = torch.randn(4, 96, 128, generator=torch.Generator().manual_seed(3)).to(DEV)
    with torch.inference_mode():
        whole = opt(x)
        again = opt(x)
        parts = torch.cat([opt(x[i:i + 1]) for i in range(4)])
    assert torch.equal(whole, again)
    assert torch.equal(whole, parts)


def test_padded_input_takes_the_layer_path():
    base, opt = _pair((2, 64, 128, 4, 128, 2, True))
    x = torch.randn(2, 64, 128, generator=torch.Generator().manual_seed(5))
    mask = torch.ones(2, 64, dtype=torch.bool)
    mask[1, 40:] = False
    calls = []
    real = tkmi.ops.small_forward
    tkmi.ops.small_forward = lambda *a, **k: calls.append(1) or real(*a, **k)
    try:
        with torch.inference_mode():
            got = opt(x.to(DEV), mask.to(DEV))
            opt(x.to(DEV))
    finally:
        tkmi.ops.small_forward = real
    assert len(calls) == 1  # only the dense call
    with torch.no_grad():
        ref = base(x, mask)
    keep = mask[..., None].expand_as(ref)
    res = ob.compare_outputs(ref[keep], got.cpu()[keep])
    assert res.passed, res.max_abs_error


@pytest.mark.parametrize("s,h", [(128, 4), (96, 1), (64, 8), (50, 2)])
def test_split_sequences_match_whole_sequence_workgroups(s, h):
    """Causal shapes with more than one 32-row block run one block per
    workgroup (K/V handed between the blocks of a sequence through the
    library's workspace) when every workgroup of the launch fits on the CUs
    at once, and one workgroup per sequence otherwise.  The same sequences
    through both launches agree bit for bit (each row's arithmetic is the
    same), and pass the oracle; a repeat of the split launch (its hand-off
    counts left at zero by the first) is identical."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    mb = (s + 31) // 32
    n_split = max(1, min(cus // mb, 64))
    n_whole = cus // mb + 1  # too many workgroups to split
    shape = (n_whole, s, 128, h, 128, 2, True)
    base, opt = _pair(shape, seed=77 + s)
    x = torch.randn(n_whole, s, 128, generator=torch.Generator().manual_seed(11 + s))
    with torch.inference_mode():
        whole = opt(x.to(DEV))
        split = opt(x[:n_split].to(DEV))
        again = opt(x[:n_split].to(DEV))
    assert torch.equal(split, again)
    assert torch.equal(split, whole[:n_split])
    with torch.no_grad():
        ref = base(x[:n_split])
    res = ob.compare_outputs(ref, split.cpu())
    print(f"s={s} h={h}: split batch {n_split}, whole-sequence batch {n_whole}, max_abs={res.max_abs_error:.3g}",
          flush=True)
    assert res.passed, (res.max_abs_error, res.failed_elements)
