"""The C project the scheduler emits for the HIP target (scheduler/codegen.py),
checked on the host: the emitted run body is the buffer plan's kernel-call list
(one cm_run_* per call, in order, with the plan's arguments and pool offsets),
the weights image is the plan's pool prefix, and the project builds with its
Makefile and with its CMakeLists.txt (reference: inference-scheduler/src/codegen/
_source.py:475-791, _header.py, _cmake.py, _test.py)."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import numpy as np
import pytest

from cormorant_amd import workloads as wl
from cormorant_amd.scheduler import BufferPlan, OnnxGraph, codegen, onnx_io as ox
from tests import onnx_models as om

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "cormorant_amd", "libcormorant_amd.so")

MODELS = {
    "mlp_b64": lambda: ox.encode_model(wl.mlp_model()),
    "conv_relu_chain": lambda: ox.encode_model(om.conv_relu_chain()),
    "broadcast_chain_bias": lambda: ox.encode_model(om.broadcast_chain_bias()),
    "gemm_chain": lambda: ox.encode_model(om.gemm_chain()),
}

_RUN = re.compile(r"RUN\((cm_run_\w+)\((.*)\)\);")


def _emitted_calls(src: str):
    return [(m.group(1), m.group(2)) for m in map(_RUN.match, (l.strip() for l in src.splitlines()))
            if m]


@pytest.mark.parametrize("name", sorted(MODELS))
def test_run_body_is_the_plan_call_list(name):
    w = codegen.ProjectWriter(OnnxGraph(MODELS[name]()), name)
    files = w.files()
    calls = _emitted_calls(files["src/inference.c"])
    plan = BufferPlan(OnnxGraph(MODELS[name]()))
    assert len(calls) == len(plan.calls)
    for (fn, args), (_, call) in zip(calls, plan.calls):
        assert fn == "cm_run_" + call.kernel
        nums = [int(v[:-1]) for v in re.findall(r"\b\d+u\b", args)]
        want = list(call.args)
        if call.kernel == "matmul_at":
            want = list(call.offsets) + want
        assert nums == want, (fn, args, call)
    # every pool view is a (offset, capacity) slot of the plan
    slots = {(st.offset, st.capacity) for st in plan.storage.values() if st.kind == "pool"}
    views = re.findall(r"\{(\d+)u, (\d+)u\},\s+/\*", files["src/inference.c"])
    assert views and all((int(o), int(c)) in slots for o, c in views)


def test_weights_image_is_the_pool_prefix():
    g = OnnxGraph(MODELS["mlp_b64"]())
    w = codegen.ProjectWriter(g, "mlp", inline_weights_max=0)
    blob = np.frombuffer(w.files()["weights.bin"], dtype="<i2")
    plan = BufferPlan(g)
    np.testing.assert_array_equal(blob, plan.pool_image()[:blob.size])
    for t in g.weight_tensors:     # every weight lies inside the file
        st = plan.storage[t.onnx_name]
        assert st.offset + st.capacity <= blob.size
    # a small model compiles its weights in
    small = codegen.ProjectWriter(OnnxGraph(MODELS["conv_relu_chain"]()), "small")
    assert small.inline and "weights.bin" not in small.files()
    assert "INFERENCE_WEIGHTS_INLINE 1" in small.files()["include/inference.h"]


@pytest.mark.skipif(not os.path.exists(LIB), reason="libcormorant_amd.so is not built")
@pytest.mark.parametrize("name", ["mlp_b64", "conv_relu_chain"])
def test_project_builds_with_make(name, tmp_path):
    codegen.write_project(OnnxGraph(MODELS[name]()), str(tmp_path), name)
    r = subprocess.run(["make", "-s", "-C", str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert (tmp_path / "libinference.a").exists() and (tmp_path / "test_inference").exists()


@pytest.mark.skipif(not os.path.exists(LIB) or shutil.which("cmake") is None,
                    reason="needs the built library and cmake")
def test_project_builds_with_cmake(tmp_path):
    src = tmp_path / "src_tree"
    codegen.write_project(OnnxGraph(MODELS["gemm_chain"]()), str(src), "gemm_chain")
    bld = tmp_path / "build"
    r = subprocess.run(["cmake", "-S", str(src), "-B", str(bld)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run(["cmake", "--build", str(bld)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert (bld / "test_inference").exists()
