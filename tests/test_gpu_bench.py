"""bench.py end to end on the GPU (in this process, short settings): exactly one JSON
line on stdout carrying the benchmark contract's fields, with self-consistent values."""
import importlib.util
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.gpu

TOP_KEYS = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
            "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
            "roofline", "cpu_baseline")


def test_bench_prints_one_contract_line(gpu, capsys, monkeypatch):
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "3", "--warmup", "1", "--no-gpt",
                                      "--no-model-ops", "--cpu-seconds", "1"])
    bench.main()
    lines = [ln for ln in capsys.readouterr().out.splitlines() if ln.strip()]
    assert len(lines) == 1, lines
    d = json.loads(lines[0])
    for k in TOP_KEYS:
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 1
    assert d["higher_is_better"] is True and d["unit"] == "TFLOP/s" and d["dtype"] == "bf16"
    assert d["vs_baseline"] is None
    assert "workload" in d["config"] and "model" not in d["config"]
    # value = algorithmic flops of one step / step time
    gflop = d["algorithmic_gflop_per_step"]
    assert d["value"] == pytest.approx(gflop / d["ms_per_step"], rel=1e-3)  # GFLOP/ms = TFLOP/s
    assert 0 < d["value"] < 2500.0

    rf = d["roofline"]
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in rf, k
    assert rf["bound"] in ("hbm", "mfma") and rf["peak"] == 2500.0
    assert 0 < rf["frac"] <= 1 and rf["frac"] == pytest.approx(rf["achieved"] / rf["peak"], rel=1e-3)

    # the HBM-cold pass of the same step, and RoPE beside its same-launch copy
    hc = d["config2_hbm_cold"]
    assert hc["sets"] * hc["set_bytes"] > 256 * 2 ** 20  # more than the Infinity Cache
    assert hc["step_us"] > 0 and set(hc["kernels"]) == {"attn_fwd", "attn_bwd_preprocess", "attn_bwd"}
    assert hc["tflops"] == pytest.approx(gflop / (hc["step_us"] * 1e-3), rel=1e-2)
    cy = d["rope"]["copy_yardstick"]
    assert cy["avg_us"] > 0 and 0 < cy["frac"] <= 1
    assert d["rope"]["frac_of_copy"] == pytest.approx(d["rope"]["frac"] / cy["frac"], rel=1e-2)

    cb = d["cpu_baseline"]
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in cb, k
    assert cb["kind"] in ("port", "reference") and cb["value"] > 0 and cb["cores"] >= 1
