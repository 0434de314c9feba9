"""GPU: the C projects the scheduler emits (scheduler/codegen.py; built by
__graft_entry__.build() under tests/c/gen/) run the MLP b64 and the
MobileNetV2-like b16 graphs through their generated inference_run, and their
test programs compare every output with the CPU oracle executing the same
kernel-call list, bit for bit."""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

import oracle
from oracle import graph_sim as gs
from cormorant_amd import workloads as wl
from cormorant_amd.scheduler import BufferPlan, OnnxGraph, onnx_io as ox
from tests.gpu_util import oracle_threads, say

pytestmark = pytest.mark.gpu
GEN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "c", "gen")

CASES = [("mlp_b64", wl.mlp_model, wl.mlp_input),
         ("mobilenet_like_b16", wl.mobilenet_model, wl.mobilenet_input)]


@pytest.mark.parametrize("name,model,inp", CASES, ids=[c[0] for c in CASES])
def test_generated_project_matches_oracle(name, model, inp, tmp_path):
    d = os.path.join(GEN, name)
    exe = os.path.join(d, "test_inference")
    assert os.path.exists(exe), "build it first: python -c 'import __graft_entry__ as g; g.build()'"
    say(f"generated C project {name}")
    plan = BufferPlan(OnnxGraph(ox.encode_model(model())))
    x = inp()
    oracle.set_threads(oracle_threads())
    want = gs.run_plan(plan, {"X": x}, threads=True)["Y"]
    xf, yf = tmp_path / "x.bin", tmp_path / "y.bin"
    np.ascontiguousarray(x, dtype="<i2").tofile(xf)
    np.ascontiguousarray(want, dtype="<i2").tofile(yf)
    r = subprocess.run([exe, os.path.join(d, "weights.bin"), str(xf), str(yf), "20"],
                       capture_output=True, text=True, timeout=120)
    say(r.stdout.strip())
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Y: PASS" in r.stdout
