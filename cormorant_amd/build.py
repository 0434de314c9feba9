"""Build libcormorant_amd.so (gfx950) in-tree with hipcc, and the cm_bench tool.

Usage: python -m cormorant_amd.build [--jobs N]

Every .hip file under csrc/ is compiled for gfx950 only and linked into one
shared library next to this file.  FP contraction is off (the pool
finalisers round exactly as written) and packed-FP32 instruction selection is
disabled.  bench_src/cm_bench.c (the per-case benchmark, a C program against
include/cormorant_amd.h) is compiled with the host C compiler and linked
against that library.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcormorant_amd.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-pass-failed",
    "-I", os.path.join(HERE, "..", "include"),
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        # keep warnings visible, but drop the host pass's note about the gfx feature flag
        lines = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l]
        if any(l.strip() for l in lines):
            sys.stderr.write("\n".join(lines) + "\n")
    return obj


def build(jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


BENCH_SRC = os.path.join(HERE, "bench_src", "cm_bench.c")
BENCH_BIN = os.path.join(HERE, "bench_src", "cm_bench")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build_bench() -> str:
    """Compile bench_src/cm_bench with gcc against the in-tree library."""
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-std=c11", "-Wall", "-Wextra",
           "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
           "-I", os.path.join(HERE, "..", "include"), BENCH_SRC,
           "-L", HERE, "-lcormorant_amd", "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/..", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-o", BENCH_BIN]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"cm_bench build failed:\n{r.stdout}\n{r.stderr}")
    return BENCH_BIN


GEN_DIR = os.path.join(HERE, "..", "tests", "c", "gen")


def build_generated_projects() -> list:
    """Emit the C projects of the two benchmark graphs (the MLP and the
    MobileNetV2-like network) with scheduler.codegen under tests/c/gen/ and build
    each with its own Makefile; the GPU tests run their test programs."""
    from . import workloads as wl
    from .scheduler import OnnxGraph, codegen, onnx_io as ox
    built = []
    for name, model in (("mlp_b64", wl.mlp_model()), ("mobilenet_like_b16", wl.mobilenet_model())):
        out = os.path.abspath(os.path.join(GEN_DIR, name))
        codegen.write_project(OnnxGraph(ox.encode_model(model)), out, name)
        r = subprocess.run(["make", "-s", "-B", "-C", out], capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"generated project {name} failed to build:\n{r.stdout}\n{r.stderr}")
        built.append(os.path.join(out, "test_inference"))
    return built


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    print(build(args.jobs))
    print(build_bench())
    for p in build_generated_projects():
        print(p)


if __name__ == "__main__":
    main()
