"""Long-sequence path (tkmi.longseq), the counterpart of src/run_case14.py.

Chain of trust, as the reference's (src/run_case14.py:1-30, 165-221):
  * at S = 100000 the case's layer shape (d_model 1024, 16 heads, ffn 1024,
    causal) is checked on 512 seeded query rows against the CPU oracle's
    sampled-row forward, which is exact for one layer (row i needs only K/V
    of rows <= i, computed for all tokens);
  * the case's two layers are checked at a feasible length against the full
    oracle;
  * chunked forwards reproduce the resident forward bit for bit (samples are
    independent), so a streamed pass inherits the resident pass's parity.
"""

from __future__ import annotations

import pytest
import torch

from oracle import baseline as ob

import tkmi
from tkmi import longseq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _pair(cfg, seed=1234):
    base = ob.build_model(cfg, seed=seed).eval()
    opt = tkmi.OptimizedTransformer(tkmi.TransformerConfig(**cfg.__dict__))
    ob.copy_model_weights(base, opt, strict=True)
    return base, opt.to(DEV).eval()


def test_case_layer_at_100k_sampled_rows():
    cfg = ob.TransformerConfig(1, 100000, 1024, 16, 1024, 1, True)
    base, opt = _pair(cfg)
    x, mask = ob.generate_random_case(cfg, seed=1234)
    rows = ob.sample_query_rows(cfg.seq_len, 512, seed=1234)
    with torch.inference_mode():
        got = opt(x.to(DEV), mask.to(DEV))[:, rows.to(DEV)].cpu()
        ref = ob.sampled_rows_forward(base, x, rows, q_chunk=256)
    res = ob.compare_outputs(ref, got)
    print(f"S=100000 sampled rows: max_abs={res.max_abs_error:.3g} failed={res.failed_elements}", flush=True)
    assert res.passed
    assert torch.isfinite(got).all()


def test_case_two_layers_at_feasible_length():
    cfg = ob.TransformerConfig(2, 2048, 1024, 16, 1024, 2, True)
    base, opt = _pair(cfg)
    x, mask = ob.generate_random_case(cfg, seed=99)
    with torch.inference_mode():
        got = opt(x.to(DEV), mask.to(DEV)).cpu()
        ref = ob.chunked_forward(base, x, q_chunk=1024)
    res = ob.compare_outputs(ref, got)
    assert res.passed, (res.max_abs_error, res.failed_elements)


@pytest.mark.parametrize("chunk", [1, 3])
def test_chunked_forward_is_bit_exact(chunk):
    cfg = tkmi.TransformerConfig(5, 1024, 256, 4, 512, 2, True)
    model = longseq.make_model(cfg, seed=5)
    x = longseq.sample_inputs(cfg, 5, 0, cfg.batch_size)
    res = longseq.check_chunks(model, x, chunk)
    assert res["bit_exact"], res


def test_sample_inputs_do_not_depend_on_chunking():
    cfg = tkmi.TransformerConfig(4, 256, 128, 4, 256, 1, True)
    whole = longseq.sample_inputs(cfg, 7, 0, 4)
    parts = torch.cat([longseq.sample_inputs(cfg, 7, s, s + 1) for s in range(4)])
    assert torch.equal(whole, parts)


@pytest.mark.parametrize("chunk", [0, 2])
def test_runner_resident_and_streamed(chunk):
    cfg = tkmi.TransformerConfig(4, 1024, 256, 4, 512, 2, True)
    summary = longseq.run(cfg, seed=3, chunk=chunk, warmup=1, repeats=2, check_chunk=2)
    assert summary["mode"].startswith("resident" if chunk == 0 else "streamed")
    assert summary["ms_median"] > 0 and len(summary["ms_all"]) == 2
    assert summary["tokens"] == 4 * 1024
    assert summary["chunk_check"]["bit_exact"]


def test_streamed_output_matches_resident():
    cfg = tkmi.TransformerConfig(4, 512, 256, 4, 512, 2, True)
    model = longseq.make_model(cfg, seed=11)
    x = longseq.sample_inputs(cfg, 11, 0, cfg.batch_size)
    with torch.inference_mode():
        want = model(x).cpu()
    host_x = torch.empty(x.shape, dtype=torch.float32, pin_memory=True)
    host_x.copy_(x)
    host_out = torch.empty(x.shape, dtype=torch.float32, pin_memory=True)
    longseq.time_streamed(model, host_x, 3, warmup=0, repeats=1, host_out=host_out)
    assert torch.equal(host_out, want)
