"""The benchmark's host-side contract, on the CPU: it refuses more than one GPU before touching the device, quotes
HBM traffic only for the kernel source it was measured on, prices every roofline against the published peaks, and
sizes its all-cores CPU baselines to at most 16 threads."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_traffic_is_quoted_only_for_the_profiled_source():
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        table = json.load(f)
    for key, e in table.items():
        src = {"k_gemm_group16 f16 step set": "scratchtape_amd/csrc/gemm_group.hip",
               "k_search": "scratchtape_amd/csrc/knn.hip", "k_search masked": "scratchtape_amd/csrc/knn.hip",
               "k_search cell-major 4096q": "scratchtape_amd/csrc/knn.hip",
               "st_knn_probe": "scratchtape_amd/csrc/knn_probe.hip", "k_attn fused step": "scratchtape_amd/csrc/attn.hip",
               "k_ln step": "scratchtape_amd/csrc/rows.hip"}[key]
        want = int(e["fetch_bytes"] + e["write_bytes"]) if e["source_sha256_16"] == bench.source_hash(src) else None
        assert bench.traffic_for(key, src) == want, key
        assert e["summary"].startswith("profiles/") and os.path.exists(os.path.join(ROOT, e["summary"])), key
    # a source other than the profiled one never inherits its figure
    assert bench.traffic_for("k_search", "scratchtape_amd/csrc/attn.hip") is None
    assert bench.traffic_for("no such kernel", "scratchtape_amd/csrc/knn.hip") is None


def test_step_set_prices_each_distinct_tensor_once():
    """The set's algorithmic bytes count X, W, dY (read by two GEMMs each) and Y, dX, dW once: 157,810,688 B, not
    the 236,716,032 B of summing every GEMM's operands."""
    ss = bench.StepSet("cpu")
    assert ss.flops == 20937965568
    assert ss.bytes == 157810688 and ss.per_gemm_bytes == 236716032
    r = bench.roofline("k", ss.flops, ss.bytes, 0.07)
    assert r["bound"] == "hbm" and r["roof_tflops"] == pytest.approx(1061.4, abs=0.1)


@pytest.mark.parametrize("flops, nbytes, bound", [(20937965568, 157810688, "hbm"), (1e12, 1e6, "mfma")])
def test_roofline_picks_the_binding_roof(flops, nbytes, bound):
    r = bench.roofline("k", flops, nbytes, 0.1, traffic=123, route="f16")
    assert r["bound"] == bound and r["traffic"] == 123
    if bound == "hbm":
        assert r["peak"] == bench.PEAK["hbm_gbs"] and r["unit"] == "GB/s"
        assert r["achieved"] == pytest.approx(nbytes / 0.1 / 1e6, abs=0.1)
    else:
        assert r["peak"] == bench.PEAK["f16"] and r["unit"] == "TFLOP/s"
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-4)


def test_published_peaks_are_the_mi355x_figures():
    assert bench.PEAK["hbm_gbs"] == 8000.0
    assert bench.PEAK["f16"] == 2500.0 and bench.PEAK["f32"] == 157.3 and bench.PEAK["i8"] == 5000.0


def test_cpu_baseline_threads_are_capped(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "3")
    assert 1 <= bench.host_threads() <= 3
    monkeypatch.setenv("OMP_NUM_THREADS", "")
    assert 1 <= bench.host_threads() <= 16
