"""C callers of the library, on the GPU.

* tests/c/capi_consumer: the INTEGRATION.md shim (inference_buf_* / run_* as
  forwards to cm_buf_* / cm_run_*) driving a small generated-runtime-style
  sequence on pool views, every VectorOP opcode, conv (standard, depthwise) and
  every pool type; it compares each output with the C oracle itself.
* cormorant_amd/bench_src/cm_bench: the per-case benchmark over the reference's
  whole case list (perf_config.json.example and the published report's extra
  rows), run with few iterations; every output it dumps is compared with the
  oracle on the same seeded inputs.
Both programs are built by __graft_entry__.build() (gcc against
include/cormorant_amd.h)."""
from __future__ import annotations

import json
import os
import subprocess

import pytest

from cormorant_amd import build as hipbuild
from cormorant_amd.bench_src import perf_cases as pc
from oracle import bench_cases as bc
from tests.gpu_util import say

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_capi_consumer_program():
    exe = os.path.join(ROOT, "tests", "c", "capi_consumer")
    assert os.path.exists(exe), "build it first: python -c 'import __graft_entry__ as g; g.build()'"
    say("C consumer program")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    say(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all cases match the oracle" in r.stdout


def test_cm_bench_every_reference_case_matches_oracle(tmp_path):
    assert os.path.exists(hipbuild.BENCH_BIN), "build it first"
    lines = []
    for c in pc.CASES:
        kind, label, args, _iters, _warm, _ = c
        lines.append(" ".join([kind, "0", label, *map(str, args), "3", "1"]))
    say(f"cm_bench over {len(lines)} cases")
    env = dict(os.environ, CM_BENCH_DUMP=str(tmp_path), CM_BENCH_SEED="7")
    r = subprocess.run([hipbuild.BENCH_BIN, "-"], input="\n".join(lines) + "\n",
                       capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-2000:]
    out = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    assert [o["label"] for o in out] == [c[1] for c in pc.CASES]
    bad = {}
    for c, o in zip(pc.CASES, out):
        assert o["seed"] == 7
        assert o["lat_ms"] > 0 and o["kernel_ms"] > 0
        n = bc.check_dump(c, str(tmp_path), seed=7)
        if n:
            bad[c[1]] = n
    assert not bad, f"outputs differing from the oracle: {bad}"
