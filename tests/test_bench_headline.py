"""bench.py's output contract, on the CPU: the headline line (printed last) stays
under its size limit with every configuration in its summary, and a multi-GPU
request is refused with a message instead of running."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _results():
    """Results shaped like a full default run (long numbers everywhere)."""
    big = 123456.789012
    ops = {k: dict(ms=0.0612345, gbs=6543.21, hbm_frac=0.817891)
           for k in ("Add", "Sub", "Mul", "Div", "Relu", "Clip06")}
    r = {"vecop": dict(ops=ops)}
    for g in ("gemm_b32_1024", "gemm_b1_4096"):
        r[g] = dict(gops=big, mfma_frac=0.361234, library_int8=dict(mfma_frac=0.416234))
    for c in ("conv_a_3x3_s1_p1", "conv_b_3x3_s2_d2_p2"):
        r[c] = dict(gops=big, mfma_frac=0.173612, frac_of_4product_roofline=0.347234,
                    packed_weights=dict(gops=big))
    for p in ("maxpool_3x3_s2", "avgpool_3x3_s2_p1_cip", "lppool_p2_2x2_s2", "globalavgpool"):
        for cv in ("conv_a", "conv_b"):
            r[f"{p}_on_{cv}"] = dict(gbs=4126.31, hbm_frac=0.515812, frac_of_copy_ceiling=0.881312)
    for o in ("56x56", "28x28"):
        r[f"pool_copy_ceiling_{o}"] = dict(gbs=4682.31, hbm_frac=0.585312)
    for g in ("mlp_b64", "mobilenet_like_b16"):
        r[g] = dict(ms_hip_graph=0.326012, images_s_hip_graph=3694744.91, roofline_frac=0.045012,
                    per_op_frac=0.088512, cpu=dict(images_s=28364.65))
    return r


def test_summary_keeps_headline_under_limit():
    results = _results()
    cases = [dict(checked_vs_oracle=True) for _ in range(49)]
    cpu = {k: dict(gops=5.123456) for k in results if k.startswith(("gemm", "conv"))}
    summary = bench.summarize(results, cases, cpu)
    # every configuration is in the digest
    assert len(summary["vecop_hbm_frac"]) == 6
    for name in results:
        if name != "vecop":
            assert name in summary, name
    assert summary["gemm_b1_4096"]["library_int8_mfma_frac"] == 0.416234
    assert summary["perf_cases"] == dict(n=49, checked_vs_oracle=True)
    # the fixed fields of the headline take ~1.4 KB; the digest must leave room
    text = json.dumps(summary, separators=(",", ":"))
    assert len(text) < bench.HEADLINE_MAX - 1600, len(text)


def test_failed_case_shows_in_summary():
    cases = [dict(checked_vs_oracle=True), dict(checked_vs_oracle=False)]
    assert bench.summarize({}, cases, {})["perf_cases"]["checked_vs_oracle"] is False


def test_multi_gpu_request_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "--gpus must be 1" in r.stderr
    assert r.stdout == ""
