"""bench.py's own logic on the CPU: the multi-GPU refusal, the algorithmic work per kernel and the roofline
arithmetic the JSON line reports (the GPU run itself is the driver's)."""
from __future__ import annotations

import importlib.util
import subprocess
import sys

import pytest

from conftest import ROOT, synth_module

spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
bench = importlib.util.module_from_spec(spec)
spec.loader.exec_module(bench)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_algorithmic_work_of_the_decode_workload():
    cfg = synth_module().CONFIGS["decode"]
    w = bench.kernel_work(cfg, active_experts=16)
    T, H, E, K, I = cfg.T, cfg.H, cfg.E, cfg.K, cfg.I
    assert (T, H, E, K, I) == (128, 2048, 16, 2, 8192)
    # gate/up: every active expert's W_gate and W_up read once, plus x
    assert w["moe_ffn_gateup_swiglu"] == (16 * 2 * 8192 * 2048 * 2 + 128 * 2048 * 2, 4 * 256 * 2048 * 8192)
    assert w["moe_ffn_gateup_swiglu"][0] == 1074266112  # the figure quoted for the roofline
    assert w["moe_ffn_down"] == (16 * 8192 * 2048 * 2 + 256 * 2048 * 2, 2 * 256 * 2048 * 8192)
    assert w["moe_combine"][0] == 256 * 2048 * 2 + 256 * 2 + 128 * 2048 * 2


def test_roofline_bound_follows_the_ridge():
    hbm = bench.roofline_for("k", 1_000_000_000, 16_000_000_000, 0.2, None)  # 16 flop/B: below the ridge
    assert hbm["bound"] == "hbm" and hbm["unit"] == "GB/s"
    assert hbm["achieved"] == pytest.approx(5000.0) and hbm["frac"] == pytest.approx(5000.0 / 8000.0, abs=1e-4)
    mfma = bench.roofline_for("k", 1_000_000_000, 1_000_000_000_000, 1.0, 123)  # 1000 flop/B: above it
    assert mfma["bound"] == "mfma" and mfma["unit"] == "TFLOP/s" and mfma["traffic"] == 123
    assert mfma["achieved"] == pytest.approx(1000.0) and mfma["frac"] == pytest.approx(0.4)
    assert bench.RIDGE == pytest.approx(312.5)
