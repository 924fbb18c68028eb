"""Host-side logic and the C ABI surface, on CPU (no kernel launches).

* the drop-in model keeps the baseline's parameter tree, seeded weights and
  strict-load compatibility (src/torch_transformer_benchmark.py:203-213,690-696);
* there is no CPU path: a CPU input raises;
* libtkmi.so loads and exports every entry point declared in include/tkmi.h;
  argument validation rejects bad calls before touching the GPU.
"""

from __future__ import annotations

import ctypes
import json
import re

import pytest
import torch

from conftest import GOLDEN_DIR, REPO
from oracle import baseline as ob

import tkmi
from tkmi import _lib

GOLD = json.loads((GOLDEN_DIR / "golden.json").read_text())
HEADER = (REPO / "include" / "tkmi.h").read_text()


def _declared_symbols():
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(tk_\w+)\s*\(", HEADER, re.M)))


def test_state_dict_keys_and_seeded_weights_match_baseline():
    cfg = tkmi.TransformerConfig(2, 16, 64, 4, 128, 2, True)
    torch.manual_seed(1234)
    opt = tkmi.OptimizedTransformer(cfg)
    base = ob.build_model(ob.TransformerConfig(**cfg.__dict__), seed=1234)
    sd_o, sd_b = opt.state_dict(), base.state_dict()
    assert list(sd_o) == list(sd_b)
    for k in sd_b:
        assert torch.equal(sd_o[k], sd_b[k]), k


def test_seeded_weights_match_reference_golden_hash():
    import hashlib

    meta = GOLD["small"]["tiny_causal"]
    torch.manual_seed(GOLD["seed"])
    opt = tkmi.OptimizedTransformer(tkmi.TransformerConfig(**meta["config"]))
    h = hashlib.sha256()
    for k, v in opt.state_dict().items():
        h.update(k.encode())
        h.update(v.numpy().tobytes())
    assert h.hexdigest() == meta["state_sha256"]


def test_strict_weight_copy_and_no_extra_state():
    cfg = ob.TransformerConfig(1, 8, 32, 2, 48, 1, False)
    base = ob.build_model(cfg)
    opt = tkmi.OptimizedTransformer(tkmi.TransformerConfig(**cfg.__dict__))
    res = ob.copy_model_weights(base, opt, strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    assert len(list(opt.buffers())) == 0


def test_forward_on_cpu_raises_no_fallback():
    cfg = tkmi.TransformerConfig(1, 8, 64, 4, 64, 1, True)
    opt = tkmi.OptimizedTransformer(cfg).eval()
    with pytest.raises(RuntimeError, match="HIP kernels only"):
        opt(torch.randn(1, 8, 64))


def test_ops_reject_cpu_tensors():
    x = torch.randn(4, 64)
    w = torch.ones(64)
    with pytest.raises(RuntimeError, match="GPU only"):
        tkmi.ops.ln_fwd(x, w, w, 1e-5)
    assert not tkmi.ops.can_fuse(x)
    assert not tkmi.ops.attention_supported(64, torch.float16, "cpu")


def test_configure_and_mask_memo():
    old = tkmi.active_settings()
    try:
        s = tkmi.configure(fused_norm=False)
        assert s.fused_norm is False and tkmi.active_settings() is s
        model = tkmi.OptimizedTransformer(tkmi.TransformerConfig(2, 4, 32, 2, 32, 1, True))
        assert model.settings.fused_norm is False
        dense = torch.ones(2, 4, dtype=torch.bool)
        padded = dense.clone()
        padded[1, 3] = False
        assert model._mask_is_dense(dense) is True
        assert model._mask_is_dense(padded) is False
        assert model._mask_is_dense(None) is True
    finally:
        tkmi.configure(**old.__dict__)


# --------------------------------------------------------------------------- #
# C ABI
# --------------------------------------------------------------------------- #


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_symbols()
    assert set(declared) == set(_lib.SIGNATURES), (declared, sorted(_lib.SIGNATURES))
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.tk_version() == _lib.ABI_VERSION


def test_every_kernel_has_a_launch_stub():
    """A kernel template whose host-side instantiation fails leaves its launch
    stub undefined (the library then fails to load on first use)."""
    import shutil
    import subprocess

    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    missing = [line for line in out.splitlines() if " U " in line and "device_stub" in line]
    assert not missing, missing[:5]


def test_capability_probes():
    lib = _lib.load()
    # the reference's rule: next_pow2(max(hd, 16)) <= 256 (src/kernels.py:96-103)
    hds = (1, 8, 16, 24, 32, 64, 100, 128, 200, 256, 257, 512)
    assert [lib.tk_attention_supported(h) for h in hds] == [1 if h <= 256 else 0 for h in hds]
    assert [lib.tk_gemm_ln_supported(n) for n in (64, 128, 256, 512, 1024)] == [0, 1, 1, 1, 0]
    # whole-forward kernel: S <= 128, d_model = ffn = 128, heads * padded head_dim = 128
    small = lib.tk_small_forward_supported
    assert [small(s, 128, 4, 32, 128) for s in (0, 1, 77, 128, 129)] == [0, 1, 1, 1, 0]
    assert [small(128, 128, h, 128 // h, 128) for h in (1, 2, 4, 8)] == [1, 1, 1, 1]
    assert small(128, 128, 16, 16, 128) == 0  # head_dim 8 pads to 16: attention width 256
    assert small(128, 256, 4, 64, 128) == 0 and small(128, 128, 4, 32, 256) == 0


@pytest.mark.parametrize(
    "fn,args,code",
    [
        ("tk_ln_cast", (None, None, None, None, 1, 4, 64, 1e-5, None, None), _lib.TK_ERR_ARG),
        ("tk_ln_cast", (8, 8, 8, 8, 1, 4, 9000, 1e-5, None, None), _lib.TK_ERR_ARG),
        ("tk_ln_cast", (8, 8, 8, 8, 7, 4, 64, 1e-5, None, None), _lib.TK_ERR_ARG),
        # tk_add_ln_cast: x of an unknown dtype, a null y, a row wider than 8192
        ("tk_add_ln_cast", (8, 5, 8, 1, 8, 8, None, 8, 1, 4, 64, 1e-5, None), _lib.TK_ERR_ARG),
        ("tk_add_ln_cast", (8, 1, None, 1, 8, 8, None, 8, 1, 4, 64, 1e-5, None), _lib.TK_ERR_ARG),
        ("tk_add_ln_cast", (8, 0, 8, 1, 8, 8, 8, 8, 1, 4, 9000, 1e-5, None), _lib.TK_ERR_ARG),
        ("tk_gemm", (16, 8, 16, 12, None, None, 0, 16, 16, 4, 4, 12, 0, None, 0, None), _lib.TK_ERR_ARG),  # lda < k
        ("tk_gemm", (17, 16, 16, 16, None, None, 0, 16, 16, 4, 4, 12, 0, None, 0, None), _lib.TK_ERR_ARG),  # odd A
        ("tk_gemm", (16, 16, 16, 16, None, None, 0, 16, 16, 4, 4, 16, 9, None, 0, None), _lib.TK_ERR_ARG),
        # a row mask needs the residual epilogue and a valid tk_row_mode
        ("tk_gemm", (16, 16, 16, 16, None, None, 0, 16, 16, 4, 4, 16, 0, 16, 1, None), _lib.TK_ERR_ARG),
        ("tk_gemm", (16, 16, 16, 16, None, 16, 16, 16, 16, 4, 4, 16, 2, 16, 7, None), _lib.TK_ERR_ARG),
        ("tk_gemm_bias_add_ln", (16, 16, 16, 16, None, 16, 16, 16, None, 16, 1, 4, 384, 16, 1e-5, None, 0, None),
         _lib.TK_ERR_UNSUPPORTED),
        ("tk_gemm_bias_add_ln", (16, 16, 16, 16, None, 16, 16, 16, None, 16, 1, 4, 128, 16, 1e-5, 16, 0, None),
         _lib.TK_ERR_ARG),
        ("tk_masked_softmax", (None, None, 1, 4, 1, None, 1, None), _lib.TK_ERR_ARG),
        ("tk_small_forward", (None, 16) + (1, 128, 128, 4, 32, 128, 4, 1) + (16,) * 14 + (1e-5, 1e-5, 1e-5, 0.17, None),
         _lib.TK_ERR_ARG),
        ("tk_small_forward", (16, 16) + (1, 256, 128, 4, 32, 128, 4, 1) + (16,) * 14 + (1e-5, 1e-5, 1e-5, 0.17, None),
         _lib.TK_ERR_UNSUPPORTED),
        ("tk_small_forward", (16, 16) + (1, 128, 128, 4, 32, 128, 0, 1) + (16,) * 14 + (1e-5, 1e-5, 1e-5, 0.17, None),
         _lib.TK_ERR_ARG),
    ],
)
def test_argument_validation_without_gpu(fn, args, code):
    lib = _lib.load()
    status = getattr(lib, fn)(*args)
    assert status == code
    assert lib.tk_last_error_string().decode()


def test_flash_rejects_bad_head_dim_without_gpu():
    lib = _lib.load()
    st = _lib.strides3((0, 0, 0))
    status = lib.tk_flash_attn_fwd(16, 16, 16, 16, 1, 1, 8, 264, st, st, st, st, 1.0, 1, None, 0, None)
    assert status == _lib.TK_ERR_UNSUPPORTED
    assert "head_dim" in lib.tk_last_error_string().decode()
    status = lib.tk_flash_attn_fwd(16, 16, 16, 16, 1, 1, 8, -1, st, st, st, st, 1.0, 1, None, 0, None)
    assert status == _lib.TK_ERR_ARG


def test_masked_softmax_checks_key_lengths_against_groups():
    """key_len is indexed per batch of heads_per_batch score groups; a short or
    mismatched key_len is rejected before any device read."""
    import tkmi.ops as ops

    scores = torch.zeros(6, 8, 8)
    with pytest.raises(ValueError, match="key_len"):
        ops.masked_softmax(scores, True, key_len=torch.tensor([8, 8], dtype=torch.int32), heads_per_batch=2)
    with pytest.raises(ValueError, match="key_len"):
        ops.masked_softmax(scores, True, key_len=torch.tensor([8, 8], dtype=torch.int32), heads_per_batch=4)
    with pytest.raises(RuntimeError, match="GPU"):  # counts fine: only the device check remains
        ops.masked_softmax(scores, True, key_len=torch.tensor([8, 8, 8], dtype=torch.int32), heads_per_batch=2)


def test_flash_rejects_short_key_mask_stride_without_gpu():
    lib = _lib.load()
    st = _lib.strides3((64, 64, 64))
    status = lib.tk_flash_attn_fwd(16, 16, 16, 16, 2, 1, 8, 64, st, st, st, st, 1.0, 1, 16, 4, None)
    assert status == _lib.TK_ERR_ARG
    assert "key_valid_stride" in lib.tk_last_error_string().decode()


# Attention instantiations the five benchmark configs dispatch:
# (kernel, head_dim, waves per workgroup, causal) -- C1, C2 (one key tile),
# C3/C5, C4.
BENCH_ATTENTION = [("flash_fwd_kernel", 32, 4, 1), ("flash_single_kernel", 64, 2, 0), ("flash_fwd_kernel", 64, 4, 1),
                   ("flash_fwd_kernel", 128, 8, 1)]


# The whole-forward kernel instantiation C1 runs (head_dim 32, causal, sequences split into
# 32-row blocks).
SMALL_FORWARD_C1 = "_ZN2tk12_GLOBAL__N_120small_forward_kernelILi128ELi128ELi128ELi32ELb1ELb1EEEvNS0_9SmallArgsE"


def test_hot_kernels_use_no_scratch():
    """A spilled accumulator costs several times the kernel's run time and no
    parity test sees it; the build's resource report must show no scratch for
    the GEMM, LayerNorm and softmax kernels, the fused QKV + attention kernel
    and the benchmarked attention and whole-forward instantiations."""
    from tkmi import build as tkbuild

    if not tkbuild.RESOURCE_PATH.exists():
        pytest.skip("library not built")
    usage = json.loads(tkbuild.RESOURCE_PATH.read_text())
    hot = [k for k in usage if any(s in k for s in ("gemm_kernel", "gemm_pf_kernel", "gemm_ln_kernel", "ln_rows_kernel",
                                                     "softmax_", "qkv_attn_kernel"))]
    assert len(hot) >= 30
    assert sum(1 for k in hot if "gemm_pf_kernel" in k) == 3  # persistent ping-pong: bias, GELU, residual
    for name, hd, nw, causal in BENCH_ATTENTION:
        hot.append(f"_ZN2tk12_GLOBAL__N_1{len(name)}{name}ILi{hd}ELi{nw}ELb{causal}ELb0EEEvNS0_8AttnArgsE")
    # every head_dim-128 instantiation, the padding-mask (key-validity) ones included:
    # the harness's --padding-ratio path at C4-like shapes
    hd128 = [k for k in usage if "flash_fwd_kernelILi128E" in k]
    assert len(hd128) == 12
    hot += hd128
    hot += [k for k in usage if "flash_generic_kernel" in k]
    # every attention instantiation (head dims 16-256, masked or not)
    hot += [k for k in usage if "flash_" in k and k not in hot]
    assert any("flash_generic_kernelILi256E" in k and "ELb1EEEv" in k for k in hot)  # the head_dim-256 vector path
    hot.append(SMALL_FORWARD_C1)
    small = [k for k in usage if "small_forward_kernel" in k and k not in hot]
    # head dims 16, 32, 64, 128: causal and not, and causal split (C1's listed above)
    assert len(small) == 11
    hot += small
    missing = [k for k in hot if k not in usage]
    assert not missing, missing
    # the 256 x 256 ping-pong GEMM instantiations (direct path, every epilogue)
    assert sum(1 for k in hot if "Li256ELi256ELi4ELi2ELi64ELi2ELb1EEE" in k and k.endswith("ELb1EEEvNS0_8GemmArgsE")) == 4
    spilled = {k: usage[k]["scratch"] for k in hot if usage[k].get("scratch", 0) > 0}
    assert not spilled, spilled


# ---------------------------------------------------------------- tooling --

def test_bench_parse_shape():
    import bench

    assert bench.parse_shape("64,128,128,4,128,4") == (64, 128, 128, 4, 128, 4, True)
    assert bench.parse_shape("2, 64, 512, 8, 2048, 4, noncausal") == (2, 64, 512, 8, 2048, 4, False)
    with pytest.raises(SystemExit):
        bench.parse_shape("1,2,3")


def test_sweep_commands_and_records():
    from tkmi import sweep

    case = {"id": 1, "batch_size": 64, "seq_len": 128, "d_model": 128, "heads": 4, "ffn_dim": 128, "layers": 4,
            "causal": True, "extra_args": ["--graph"]}
    cmd = sweep.case_command(case, ["--steps", "5"])
    assert cmd[1].endswith("bench.py") and cmd[2:4] == ["--shape", "64,128,128,4,128,4,causal"]
    assert cmd[-3:] == ["--steps", "5", "--graph"]  # passthrough first, then the case's own flags
    long_case = dict(case, id=14, runner="longseq", extra_args=[])
    assert sweep.case_command(long_case, ["--steps", "5"])[1:3] == ["-m", "tkmi.longseq"]
    line = {"ms_per_step": 0.25, "tokens_per_s": 3.2e7, "value": 0.0625, "roofline": {"frac": 0.1},
            "input_dtype": "float32", "device": "gpu", "cpu_baseline": {"forward_ms": 50.0, "cores": 16, "sample": "s"},
            "parity": {"passed": True, "max_abs": 1e-3, "failed": 0, "elements": 10}}
    rec = sweep.parse_result(case, sweep._last_json("noise\n" + json.dumps(line) + "\n"))
    assert rec["optimized"]["median_ms"] == 0.25 and rec["speedup"] == 200.0
    assert rec["accuracy"]["passed"] and sweep.classify(0, rec, False) == "ok"
    bad = dict(rec, accuracy=dict(rec["accuracy"], passed=False))
    assert sweep.classify(0, bad, False) == "accuracy_failed"
    assert sweep.classify(1, rec, False) == "error" and sweep.classify(0, rec, True) == "timeout"
    assert sweep.classify(0, {}, False) == "error"


def test_dispatch_table_keeps_fastest_passing_run(tmp_path):
    from tkmi import dispatch

    case = {"id": 1, "batch_size": 64, "seq_len": 128, "d_model": 128, "heads": 4, "ffn_dim": 128, "layers": 4,
            "causal": True}
    def results(name, passthrough, ms, status="ok"):
        path = tmp_path / name
        path.write_text(json.dumps({"schema": 1, "passthrough_args": passthrough,
                                    "cases": [{"case": case, "status": status, "optimized": {"median_ms": ms}}]}))
        return path
    paths = [results("eager.json", [], 0.27), results("graph.json", ["--graph"], 0.12),
             results("broken.json", ["--unfused-norm"], 0.01, status="accuracy_failed")]
    table = dispatch.build_table(paths)
    assert len(table["shapes"]) == 1
    entry = table["shapes"][0]
    assert entry["settings"] == {"graph": True, "fused_norm": True} and entry["median_ms"] == 0.12
    assert dispatch.settings_for(table, 64, 128, 128, 4, 128, 4, True) == {"graph": True, "fused_norm": True}
    assert dispatch.settings_for(table, 64, 128, 128, 4, 128, 4, False) is None


def test_shape_tables_are_well_formed():
    from tkmi import sweep

    for name in ("shapes.json", "baseline.json"):
        table = json.loads((sweep.PKG / "configs" / name).read_text())
        ids = [c["id"] for c in table["cases"]]
        assert len(ids) == len(set(ids))
        for c in table["cases"]:
            assert c["d_model"] % c["heads"] == 0
    appendix = json.loads((sweep.PKG / "configs" / "shapes.json").read_text())["cases"]
    assert len(appendix) == 14 and appendix[-1]["runner"] == "longseq"
