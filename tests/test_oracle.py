"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Each oracle function is checked against something that would catch a
plausible mistake in it:
  * golden vectors written from the reference itself (seeded weight hashes,
    inputs, outputs, accuracy-rule verdicts) -- tests/golden/make_golden.py;
  * the independent float64 twin (oracle/twin64.py) on tiny shapes;
  * closed forms and brute force (LayerNorm, GELU, softmax, attention);
  * invariants (causal rows ignore future keys, softmax rows sum to 1,
    chunked == unchunked);
  * planted mistakes: a perturbed oracle must FAIL the golden checks.
"""

from __future__ import annotations

import hashlib
import json
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN_DIR, seeded
from oracle import baseline as ob
from oracle import twin64

GOLD = json.loads((GOLDEN_DIR / "golden.json").read_text())
ARR = np.load(GOLDEN_DIR / "golden.npz")  # allow_pickle defaults to False


def _state_hash(module) -> str:
    h = hashlib.sha256()
    for key, value in module.state_dict().items():
        h.update(key.encode())
        h.update(value.detach().contiguous().cpu().numpy().tobytes())
    return h.hexdigest()


def _cfg(d):
    return ob.TransformerConfig(**d)


# --------------------------------------------------------------------------- #
# Golden vectors from the reference
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("name", sorted(GOLD["small"]))
def test_seeded_weights_match_reference(name):
    cfg = _cfg(GOLD["small"][name]["config"])
    model = ob.build_model(cfg, seed=GOLD["seed"])
    assert _state_hash(model) == GOLD["small"][name]["state_sha256"]


@pytest.mark.parametrize("name", sorted(GOLD["full"]))
def test_seeded_weights_and_inputs_match_reference_full_configs(name):
    entry = GOLD["full"][name]
    cfg = _cfg(entry["config"])
    model = ob.build_model(cfg, seed=GOLD["seed"])
    assert _state_hash(model) == entry["state_sha256"]
    del model
    x, mask = ob.generate_random_case(cfg, seed=GOLD["seed"])
    assert hashlib.sha256(x.numpy().tobytes()).hexdigest() == entry["x_sha256"]
    assert bool(mask.all())


@pytest.mark.parametrize("name", sorted(GOLD["small"]))
def test_forward_matches_reference_output(name):
    meta = GOLD["small"][name]
    cfg = _cfg(meta["config"])
    model = ob.build_model(cfg, seed=GOLD["seed"]).eval()
    x, mask = ob.generate_random_case(cfg, seed=GOLD["seed"], padding_ratio=meta["padding_ratio"])
    assert torch.equal(x, torch.from_numpy(ARR[f"{name}.x"]))
    assert torch.equal(mask, torch.from_numpy(ARR[f"{name}.mask"]))
    with torch.inference_mode():
        out = model(x, mask)
    want = torch.from_numpy(ARR[f"{name}.out"])
    # Same torch CPU kernels as the reference run: agreement at fp32 rounding
    # level (bit-exact on the machine that wrote the fixture).
    torch.testing.assert_close(out, want, atol=2e-6, rtol=0)


def test_compare_outputs_matches_reference_verdicts():
    ref = torch.from_numpy(ARR["cmp.ref"])
    opt = torch.from_numpy(ARR["cmp.opt"])
    res = ob.compare_outputs(ref, opt, rtol=0.02, atol=0.002)
    want = GOLD["compare_outputs"]
    assert res.passed == want["passed"]
    assert res.failed_elements == want["failed_elements"]
    assert res.failed_feature_dims == want["failed_feature_dims"]


def test_compare_outputs_branches():
    # abs branch, rel branch, both fail, non-finite fail
    ref = torch.tensor([1.0, 0.05, 10.0, 0.0, 1.0])
    opt = torch.tensor([1.0019, 0.0519, 10.19, 0.0021, float("nan")])
    res = ob.compare_outputs(ref, opt)
    assert res.failed_elements == 2 and res.failed_feature_dims == [3, 4]
    # the relative term uses |ref|, not |opt|
    res = ob.compare_outputs(torch.tensor([-1.0]), torch.tensor([-1.019]))
    assert res.passed


# --------------------------------------------------------------------------- #
# Planted mistakes must fail the golden checks
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize(
    "mutation",
    ["drop_out_bias", "swap_qk", "no_causal", "ln_eps", "gelu_tanh"],
)
def test_planted_oracle_mistakes_are_caught(mutation, monkeypatch):
    name = "tiny_causal"
    meta = GOLD["small"][name]
    cfg = _cfg(meta["config"])
    model = ob.build_model(cfg, seed=GOLD["seed"]).eval()
    x = torch.from_numpy(ARR[f"{name}.x"])
    want = torch.from_numpy(ARR[f"{name}.out"])
    if mutation == "drop_out_bias":
        with torch.no_grad():
            model.layers[0].attention.out_proj.bias.zero_()
    elif mutation == "swap_qk":
        for layer in model.layers:
            a = layer.attention
            a.q_proj, a.k_proj = a.k_proj, a.q_proj
    elif mutation == "no_causal":
        model.config = ob.TransformerConfig(**{**meta["config"], "causal": False})
    elif mutation == "ln_eps":
        model.final_norm.eps = 1e-3
    elif mutation == "gelu_tanh":
        real = F.gelu
        monkeypatch.setattr(ob.F, "gelu", lambda t, approximate="none": real(t, approximate="tanh"))
    with torch.inference_mode():
        out = model(x)
    fails, _ = (ob.compare_outputs(want, out, atol=1e-5, rtol=0).failed_elements, None)
    assert fails > 0, f"mutation {mutation} was not detected"


# --------------------------------------------------------------------------- #
# float64 twin
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("name", ["tiny_causal", "tiny_full", "c1_b1"])
def test_oracle_matches_float64_twin(name):
    meta = GOLD["small"][name]
    cfg = _cfg(meta["config"])
    model = ob.build_model(cfg, seed=GOLD["seed"]).eval()
    x = torch.from_numpy(ARR[f"{name}.x"])
    with torch.inference_mode():
        out32 = model(x)
    out64 = twin64.forward64(model.state_dict(), cfg, x)
    err = (out32.double() - out64).abs().max().item()
    assert err < 2e-5, err
    # and the reference output itself sits equally close to the twin
    ref_err = (torch.from_numpy(ARR[f"{name}.out"]).double() - out64).abs().max().item()
    assert ref_err < 2e-5, ref_err


# --------------------------------------------------------------------------- #
# Per-kernel references vs closed forms / brute force
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("d", [32, 64, 100, 128, 1024])
def test_layer_norm_ref_closed_form(d):
    x = seeded(48, d, seed=d) * 3 + 0.5
    w = seeded(d, seed=d + 1, scale=0.5) + 1.0
    b = seeded(d, seed=d + 2, scale=0.5)
    got = ob.layer_norm_ref(x, w, b, 1e-5)
    xd = x.double()
    mean = xd.mean(-1, keepdim=True)
    var = ((xd - mean) ** 2).mean(-1, keepdim=True)  # population variance
    want = (xd - mean) / torch.sqrt(var + 1e-5) * w.double() + b.double()
    assert (got.double() - want).abs().max() < 1e-5
    s, h = ob.add_layer_norm_ref(x, x.half(), w, b, 1e-5, torch.float16)
    assert torch.equal(s, x + x.half().float()) and h.dtype == torch.float16


def test_gelu_ref_closed_form():
    x = torch.linspace(-6, 6, 1001)
    want = torch.tensor([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.tolist()])
    assert (ob.gelu_ref(x) - want).abs().max() < 1e-6


def _attention_brute(q, k, v, scale, causal):
    b, h, s, hd = q.shape
    out = torch.zeros(b, s, h * hd, dtype=torch.float64)
    for bi in range(b):
        for hi in range(h):
            for i in range(s):
                lim = i + 1 if causal else s
                sc = [float(q[bi, hi, i].double() @ k[bi, hi, j].double()) * scale for j in range(lim)]
                m = max(sc)
                e = [math.exp(t - m) for t in sc]
                z = sum(e)
                row = sum((e[j] / z) * v[bi, hi, j].double() for j in range(lim))
                out[bi, i, hi * hd : (hi + 1) * hd] = row
    return out


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 2, 9, 8), (2, 1, 5, 16)])
def test_attention_ref_brute_force(shape, causal):
    b, h, s, hd = shape
    q, k, v = (seeded(*shape, seed=i) for i in (1, 2, 3))
    got = ob.attention_ref(q, k, v, hd ** -0.5, causal)
    want = _attention_brute(q, k, v, hd ** -0.5, causal)
    assert (got.double() - want).abs().max() < 1e-5


def test_masked_softmax_ref_invariants():
    s = seeded(3, 7, 7, seed=5)
    p = ob.masked_softmax_ref(s, causal=True)
    torch.testing.assert_close(p.sum(-1), torch.ones(3, 7))
    assert torch.all(p.triu(1) == 0)
    kv = torch.tensor([True] * 5 + [False] * 2)
    p2 = ob.masked_softmax_ref(s, causal=False, key_valid=kv)
    assert torch.all(p2[..., 5:] == 0)
    torch.testing.assert_close(p2.sum(-1), torch.ones(3, 7))


def test_causal_rows_ignore_future_keys():
    q, k, v = (seeded(1, 2, 12, 8, seed=i) for i in (7, 8, 9))
    base = ob.attention_ref(q, k, v, 8 ** -0.5, True)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 6:] += 3.0
    v2[:, :, 6:] -= 2.0
    alt = ob.attention_ref(q, k2, v2, 8 ** -0.5, True)
    assert torch.equal(base[:, :6], alt[:, :6])
    assert not torch.allclose(base[:, 6:], alt[:, 6:])


# --------------------------------------------------------------------------- #
# Long-sequence references (chain of trust, src/run_case14.py:165-221)
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("causal", [True, False])
def test_chunked_forward_equals_baseline(causal):
    cfg = ob.TransformerConfig(2, 96, 64, 4, 128, 2, causal)
    model = ob.build_model(cfg).eval()
    x, _ = ob.generate_random_case(cfg)
    with torch.inference_mode():
        full = model(x)
        chunked = ob.chunked_forward(model, x, q_chunk=40)
    assert (full - chunked).abs().max() < ob.ATOL / 20


def test_sampled_rows_forward_equals_baseline_rows():
    cfg = ob.TransformerConfig(2, 128, 64, 4, 128, 1, True)
    model = ob.build_model(cfg).eval()
    x, _ = ob.generate_random_case(cfg)
    rows = ob.sample_query_rows(cfg.seq_len, 20)
    with torch.inference_mode():
        full = model(x)
        part = ob.sampled_rows_forward(model, x, rows, q_chunk=7)
    assert (full[:, rows] - part).abs().max() < ob.ATOL / 20


def test_flop_counts():
    c3 = ob.TransformerConfig(8, 2048, 1024, 16, 4096, 6, True)
    assert abs(ob.gemm_flops(c3) / 6 - 412.3e9) / 412.3e9 < 1e-3
    assert abs(ob.attention_flops(c3) / 6 - 68.8e9) / 68.8e9 < 2e-3
