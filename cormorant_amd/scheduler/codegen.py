"""C project emission for the HIP target.

The reference scheduler's last stage writes a C project that runs the model
on the KV260 kernels: include/inference.h (data type, size macros, the DMA
buffer API, inference_init / inference_run / inference_deinit), src/inference.c
(one pool allocation with a view per weight and intermediate, the weights
copied in once, one run_* line per scheduled kernel call, host syncs only at
the graph's inputs and outputs), CMakeLists.txt and a test program
(inference-scheduler/src/codegen/_header.py, _source.py:475-791, _cmake.py,
_test.py).  This module writes the same project for the MI355X library:

* ``include/inference.h`` -- ``Data_t`` = int16 Q8.8, ``INFERENCE_<T>_SIZE``
  (buffer elements, padding included) and the layout of every graph input and
  output, ``INFERENCE_BUF_POOL_SIZE_BYTES``, ``inference_buf_t`` = ``cm_buf_t``
  and the ``inference_buf_*`` functions over the library's buffer API, and
  ``inference_init`` / ``inference_run`` / ``inference_deinit``;
* ``src/inference.c`` -- the pool allocation and its views, the weights (a C
  array for small models, else the file ``weights.bin`` read at init: the
  reference's ``_load_weight`` path for large weights), a split-K workspace
  sized at init from ``cm_*_workspace_size`` over the model's calls, and one
  ``cm_run_*`` call per kernel call of the buffer plan, in order -- the same
  calls, arguments and pool offsets the scheduler session runs unfused;
* ``test/test_inference.c`` -- loads inputs and expected outputs (raw int16,
  logical order) from files, runs the model, compares bit for bit, times it;
* ``Makefile`` and ``CMakeLists.txt`` -- build ``libinference.a`` and the test
  program against ``libcormorant_amd.so``.

Differences from the reference's output: there are no UIO device names to pass
(``inference_init`` takes the weights file instead, NULL when the weights are
compiled in); ``inference_run`` returns 0 or the first failing call's negative
status instead of nothing; buffers carry no reference count, because the plan
already resolves output alias chains to the caller's buffer (the reference
swaps pointers and retains the caller's buffer around the calls).
"""
from __future__ import annotations

import os
from typing import Dict, List, Optional, Tuple, Union

import numpy as np

from .graph import OnnxGraph
from .nodes import KernelCall
from .plan import BufferPlan
from .tensor import BYTES_PER_ELEM, POOL_ALIGN_BYTES, c_identifier

INLINE_WEIGHTS_MAX = 1 << 16     # elements: larger weight images go to weights.bin

_HEADER_API = r"""
/* ------------------------------------------------------------------ buffers */
/* DMA-capable buffer handle (the library's cm_buf_t: `host` is the CPU-side
 * mirror, the reference's `virt`; `dev` the device address, its `phys`). */
typedef cm_buf_t inference_buf_t;

/* Allocate a buffer of n_elem Data_t elements; NULL on failure. */
inference_buf_t *inference_buf_alloc(unsigned n_elem);
/* Release an owning buffer (views: no-op). */
void inference_buf_free(inference_buf_t *buf);
/* CPU-accessible pointer to the buffer's host mirror. */
Data_t *inference_buf_ptr(inference_buf_t *buf);
/* Device address of the buffer's first element. */
uint64_t inference_buf_phys(const inference_buf_t *buf);
/* Number of Data_t elements the buffer holds. */
unsigned inference_buf_count(const inference_buf_t *buf);
/* *view = count_elems elements of *base from offset_elems on (shares memory). */
void inference_buf_init_view(inference_buf_t *view, inference_buf_t *base,
                             unsigned offset_elems, unsigned count_elems);
/* Host mirror -> device (stream-ordered). */
void inference_buf_sync_to_device(inference_buf_t *buf);
/* Device -> host mirror; returns when the data is there. */
void inference_buf_sync_from_device(inference_buf_t *buf);

/* ---------------------------------------------------------------- inference */
/* inference_init() -- allocate the pool and the split-K workspace, load the
 * weights (from weights_path, or the compiled-in image when it is NULL and the
 * project has one) and copy them to the device.  0 on success. */
int inference_init(const char *weights_path);

/* inference_deinit() -- release every buffer inference_init allocated. */
void inference_deinit(void);
"""


def _c_array(values: np.ndarray, per_line: int = 16) -> str:
    vals = [str(int(v)) for v in np.asarray(values, dtype=np.int16).reshape(-1)]
    lines = [", ".join(vals[i:i + per_line]) for i in range(0, len(vals), per_line)]
    return "    " + ",\n    ".join(lines)


class ProjectWriter:
    """Emits the C project of one model (an OnnxGraph, or ONNX bytes / path)."""

    def __init__(self, model: Union[OnnxGraph, bytes, str], name: str = "model",
                 inline_weights_max: int = INLINE_WEIGHTS_MAX,
                 cormorant_root: Optional[str] = None) -> None:
        self.graph = model if isinstance(model, OnnxGraph) else OnnxGraph(model)
        self.plan = BufferPlan(self.graph)
        self.name = name
        self.root = os.path.abspath(cormorant_root or os.path.join(
            os.path.dirname(os.path.abspath(__file__)), "..", ".."))
        wt = [self.plan.storage[t.onnx_name] for t in self.graph.weight_tensors]
        self.weights_end = max((st.offset + st.capacity for st in wt), default=0)
        self.inline = self.weights_end <= inline_weights_max
        self._views: Dict[Tuple[int, int], int] = {}
        self._view_names: Dict[int, str] = {}

    # ----------------------------------------------------------- tensor refs
    def _io_param(self, kind: str, key: str) -> str:
        return f"{'in' if kind == 'input' else 'out'}_{c_identifier(key)}"

    def _ref(self, name: Optional[str]) -> str:
        """C expression of the buffer (pointer) that backs tensor `name`."""
        if name is None:
            return "NULL"
        st = self.plan.storage[name]
        if st.kind in ("input", "output"):
            assert st.offset == 0
            return self._io_param(st.kind, st.key)
        key = (st.offset, st.capacity)
        if key not in self._views:
            self._views[key] = len(self._views)
            self._view_names[self._views[key]] = name
        return f"&s_view[{self._views[key]}]"

    def _call_line(self, call: KernelCall) -> str:
        t, a = call.tensors, ", ".join(f"{v}u" for v in call.args)
        if call.kernel == "op":
            return f"cm_run_op({self._ref(t[0])}, {self._ref(t[1])}, {self._ref(t[2])}, {a})"
        if call.kernel == "matmul":
            return f"cm_run_matmul({self._ref(t[0])}, {self._ref(t[1])}, {self._ref(t[2])}, {a})"
        if call.kernel == "matmul_at":
            o = call.offsets
            return (f"cm_run_matmul_at({self._ref(t[0])}, {o[0]}u, {self._ref(t[1])}, {o[1]}u, "
                    f"{self._ref(t[2])}, {o[2]}u, {a})")
        if call.kernel == "conv":
            return (f"cm_run_conv({self._ref(t[0])}, {self._ref(t[1])}, {self._ref(t[2])}, "
                    f"{self._ref(t[3])}, {a})")
        if call.kernel == "pool":
            return f"cm_run_pool({self._ref(t[0])}, {self._ref(t[1])}, {a})"
        raise ValueError(f"unknown kernel '{call.kernel}'")

    def _ws_line(self, call: KernelCall) -> Optional[str]:
        a = ", ".join(f"{v}u" for v in call.args)
        if call.kernel in ("matmul", "matmul_at"):
            return f"cm_matmul_workspace_size({a})"
        if call.kernel == "conv":
            return f"cm_conv_workspace_size({a})"
        return None

    # ---------------------------------------------------------------- header
    def header(self) -> str:
        g, plan = self.graph, self.plan
        out = [f"/* inference.h -- generated for model '{self.name}' by cormorant_amd.scheduler."
               "codegen:",
               " * its graph run on one MI355X through libcormorant_amd (include/cormorant_amd.h).",
               " * Counterpart of the reference's generated include/inference.h",
               " * (inference-scheduler/src/codegen/_header.py). */",
               "#ifndef INFERENCE_H", "#define INFERENCE_H", "",
               "#include <stdint.h>", "#include \"cormorant_amd.h\"", "",
               "#ifdef __cplusplus", "extern \"C\" {", "#endif", "",
               "/* ap_fixed<16,8> stored as raw int16 (value = raw / 256) */",
               "typedef int16_t Data_t;",
               f"#define INFERENCE_BYTES_PER_ELEM  {BYTES_PER_ELEM}u",
               f"#define INFERENCE_ALIGN_BYTES     {POOL_ALIGN_BYTES}u", "",
               "/* Graph inputs and outputs: SIZE = buffer elements (padding included);",
               " * the data sit in N_CHUNKS blocks of CHUNK elements STRIDE apart (one",
               " * block when flat), zeros between them; NUMEL = logical elements. */"]
        for t in g.input_tensors + g.output_tensors:
            lay = plan.layouts[t.onnx_name]
            u = t.c_name.upper()
            out.append(f"#define INFERENCE_{u}_SIZE      {lay.alloc}u   /* shape {list(t.shape)} */")
            out.append(f"#define INFERENCE_{u}_NUMEL     {lay.numel}u")
            out.append(f"#define INFERENCE_{u}_N_CHUNKS  {lay.n_chunks}u")
            out.append(f"#define INFERENCE_{u}_CHUNK     {lay.chunk}u")
            out.append(f"#define INFERENCE_{u}_STRIDE    {lay.stride}u")
        out += ["", "/* One device allocation holds the weights and every intermediate. */",
                f"#define INFERENCE_BUF_POOL_SIZE_BYTES  {plan.pool_elems * BYTES_PER_ELEM}u",
                f"#define INFERENCE_N_INPUTS   {len(g.input_tensors)}u",
                f"#define INFERENCE_N_OUTPUTS  {len(g.output_tensors)}u",
                f"#define INFERENCE_WEIGHTS_INLINE {1 if self.inline else 0}",
                _HEADER_API]
        params = [f"inference_buf_t *{self._io_param('input', t.onnx_name)}" for t in g.input_tensors]
        params += [f"inference_buf_t *{self._io_param('output', t.onnx_name)}" for t in g.output_tensors]
        out.append("/* inference_run() -- run the graph: inputs synced to the device, every")
        out.append(" * kernel call queued in order, outputs synced back (the only host waits).")
        for t in g.input_tensors:
            out.append(f" *   {self._io_param('input', t.onnx_name):<24} [in]  INFERENCE_{t.c_name.upper()}_SIZE elements")
        for t in g.output_tensors:
            out.append(f" *   {self._io_param('output', t.onnx_name):<24} [out] INFERENCE_{t.c_name.upper()}_SIZE elements")
        out.append(" * Returns 0, or the first failing call's negative CM_ERR_* status. */")
        out.append("int inference_run(" + ", ".join(params) + ");")
        out += ["", "#ifdef __cplusplus", "}", "#endif", "", "#endif /* INFERENCE_H */", ""]
        return "\n".join(out)

    # ---------------------------------------------------------------- source
    def source(self) -> str:
        g, plan = self.graph, self.plan
        body: List[str] = []
        ws_terms: List[str] = []
        for idx, call in plan.calls:
            node = g.nodes[idx].onnx_node if idx < len(g.nodes) else None
            what = f"{node.op_type} '{node.name}'" if node is not None else "graph-output copy"
            body.append(f"    /* [{idx}] {what}: {call} */")
            body.append(f"    RUN({self._call_line(call)});")
            w = self._ws_line(call)
            if w is not None:
                ws_terms.append(w)
        views = sorted(self._views.items(), key=lambda kv: kv[1])
        out = [f"/* inference.c -- generated for model '{self.name}' by cormorant_amd.scheduler."
               "codegen.",
               " * Counterpart of the reference's generated src/inference.c",
               " * (inference-scheduler/src/codegen/_source.py:475-791). */",
               "#include <stdio.h>", "#include <stdlib.h>", "#include <string.h>", "",
               "#include \"inference.h\"", "",
               f"#define POOL_ELEMS     {plan.pool_elems}u",
               f"#define WEIGHTS_ELEMS  {self.weights_end}u   /* pool prefix holding the weights */",
               f"#define N_VIEWS        {len(views)}u", ""]
        if self.inline:
            img = plan.pool_image()[:self.weights_end]
            out.append("static const int16_t s_weights[WEIGHTS_ELEMS + 1] = {")
            out.append(_c_array(np.concatenate([img, np.zeros(1, np.int16)])))
            out.append("};")
            out.append("")
        out.append("/* views of the pool: (element offset, elements), one per storage slot")
        out.append(" * (a weight, or intermediates whose live ranges never overlap) */")
        out.append("static const uint32_t s_view_at[N_VIEWS + 1][2] = {")
        for (off, cap), i in views:
            out.append(f"    {{{off}u, {cap}u}},   /* [{i}] {self._view_names[i]} */")
        out.append("    {0u, 0u}")
        out.append("};")
        out += ["", "static inference_buf_t *s_alloc_pool;", "static inference_buf_t *s_workspace;",
                f"static inference_buf_t s_view[N_VIEWS + 1];", "",
                "/* ---- buffer API over the library's (reference names) ---- */",
                "inference_buf_t *inference_buf_alloc(unsigned n_elem) { return cm_buf_alloc(n_elem); }",
                "void inference_buf_free(inference_buf_t *buf) { cm_buf_free(buf); }",
                "Data_t *inference_buf_ptr(inference_buf_t *buf) { return cm_buf_ptr(buf); }",
                "uint64_t inference_buf_phys(const inference_buf_t *buf) { return (uint64_t)(uintptr_t)buf->dev; }",
                "unsigned inference_buf_count(const inference_buf_t *buf) { return cm_buf_count(buf); }",
                "void inference_buf_init_view(inference_buf_t *view, inference_buf_t *base,",
                "                             unsigned offset_elems, unsigned count_elems)",
                "{ cm_buf_init_view(view, base, offset_elems, count_elems); }",
                "void inference_buf_sync_to_device(inference_buf_t *buf) { cm_buf_sync_to_device(buf); }",
                "void inference_buf_sync_from_device(inference_buf_t *buf) { cm_buf_sync_from_device(buf); }",
                "",
                "static size_t max_size(size_t a, size_t b) { return a > b ? a : b; }", "",
                "int inference_init(const char *weights_path)",
                "{",
                "    int rc = cm_buf_pool_init();",
                "    if (rc != 0) return rc;",
                "    s_alloc_pool = cm_buf_alloc(POOL_ELEMS);",
                "    if (!s_alloc_pool) { rc = CM_ERR_NOMEM; goto fail; }",
                "    for (uint32_t i = 0; i < N_VIEWS; ++i)",
                "        cm_buf_init_view(&s_view[i], s_alloc_pool, s_view_at[i][0], s_view_at[i][1]);",
                "    /* weights: the pool's first WEIGHTS_ELEMS elements, in one copy */",
                "    memset(cm_buf_ptr(s_alloc_pool), 0, (size_t)POOL_ELEMS * sizeof(Data_t));"]
        if self.inline:
            out += ["    if (!weights_path) {",
                    "        memcpy(cm_buf_ptr(s_alloc_pool), s_weights, (size_t)WEIGHTS_ELEMS * sizeof(Data_t));",
                    "    } else {"]
        else:
            out += ["    if (!weights_path) { rc = CM_ERR_INVALID; goto fail; }",
                    "    {"]
        out += ["        FILE *f = fopen(weights_path, \"rb\");",
                "        if (!f) { fprintf(stderr, \"inference_init: cannot open %s\\n\", weights_path); rc = CM_ERR_INVALID; goto fail; }",
                "        size_t got = fread(cm_buf_ptr(s_alloc_pool), sizeof(Data_t), WEIGHTS_ELEMS, f);",
                "        fclose(f);",
                "        if (got != WEIGHTS_ELEMS) {",
                "            fprintf(stderr, \"inference_init: %s holds %zu of %u elements\\n\", weights_path, got, WEIGHTS_ELEMS);",
                "            rc = CM_ERR_INVALID; goto fail;",
                "        }",
                "    }",
                "    rc = cm_buf_sync_to_device(s_alloc_pool);",
                "    if (rc != 0) goto fail;",
                "    /* split-K workspace: the largest any call of the model uses (calls run",
                "     * one after another on one stream, so they share it) */",
                "    {",
                "        size_t ws = 0;"]
        for w in ws_terms:
            out.append(f"        ws = max_size(ws, {w});")
        out += ["        if (ws) {",
                "            s_workspace = cm_buf_alloc((uint32_t)((ws + 1) / 2));",
                "            if (!s_workspace) { rc = CM_ERR_NOMEM; goto fail; }",
                "            rc = cm_set_workspace(cm_buf_dev(s_workspace), ws);",
                "            if (rc != 0) goto fail;",
                "        }",
                "    }",
                "    return 0;",
                "fail:",
                "    inference_deinit();",
                "    return rc;",
                "}", "",
                "void inference_deinit(void)",
                "{",
                "    cm_set_workspace(NULL, 0);",
                "    if (s_workspace) { cm_buf_free(s_workspace); s_workspace = NULL; }",
                "    if (s_alloc_pool) { cm_buf_free(s_alloc_pool); s_alloc_pool = NULL; }",
                "    cm_buf_pool_deinit();",
                "}", "",
                "/* the first failing call's status is kept; later calls still run (as the",
                " * reference's void helpers do) so that the stream's order is unchanged */",
                "#define RUN(call) do { int rc_ = (call); if (rc_ && !rc) rc = rc_; } while (0)", ""]
        params = [f"inference_buf_t *{self._io_param('input', t.onnx_name)}" for t in g.input_tensors]
        params += [f"inference_buf_t *{self._io_param('output', t.onnx_name)}" for t in g.output_tensors]
        out.append("int inference_run(" + ", ".join(params) + ")")
        out.append("{")
        out.append("    int rc = 0;")
        for t in g.input_tensors:
            out.append(f"    RUN(cm_buf_sync_to_device({self._io_param('input', t.onnx_name)}));")
        out += body
        for t in g.output_tensors:
            out.append(f"    RUN(cm_buf_sync_from_device({self._io_param('output', t.onnx_name)}));")
        out += ["    return rc;", "}", ""]
        return "\n".join(out)

    # ------------------------------------------------------------------ test
    def test_program(self) -> str:
        g = self.graph
        ins, outs = g.input_tensors, g.output_tensors
        out = [f"/* test_inference.c -- generated for model '{self.name}': the counterpart of the",
               " * reference's generated test program (inference-scheduler/src/codegen/_test.py).",
               " * usage: test_inference WEIGHTS|- IN.bin... EXPECTED.bin... [ITERATIONS]",
               " *   raw little-endian int16 files in logical (ONNX) order, inputs then",
               " *   expected outputs in graph order; '-' = the compiled-in weights.",
               " * Prints one line per output and the mean time of inference_run; exit",
               " * status 0 when every output matches bit for bit. */",
               "#define _POSIX_C_SOURCE 199309L   /* clock_gettime */",
               "#include <stdio.h>", "#include <stdlib.h>", "#include <string.h>", "#include <time.h>", "",
               "#include \"inference.h\"", "",
               "typedef struct { const char *name; unsigned size, numel, n_chunks, chunk, stride; } io_t;",
               "static const io_t k_in[] = {"]
        for t in ins:
            u = t.c_name.upper()
            out.append(f"    {{\"{t.onnx_name}\", INFERENCE_{u}_SIZE, INFERENCE_{u}_NUMEL, "
                       f"INFERENCE_{u}_N_CHUNKS, INFERENCE_{u}_CHUNK, INFERENCE_{u}_STRIDE}},")
        out.append("};")
        out.append("static const io_t k_out[] = {")
        for t in outs:
            u = t.c_name.upper()
            out.append(f"    {{\"{t.onnx_name}\", INFERENCE_{u}_SIZE, INFERENCE_{u}_NUMEL, "
                       f"INFERENCE_{u}_N_CHUNKS, INFERENCE_{u}_CHUNK, INFERENCE_{u}_STRIDE}},")
        out.append("};")
        out += [r"""
/* buffer position of logical element i */
static size_t pos_of(const io_t *t, size_t i)
{ return t->n_chunks > 1 ? (i / t->chunk) * t->stride + i % t->chunk : i; }

static int16_t *load(const char *path, size_t n)
{
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "cannot open %s\n", path); exit(2); }
    int16_t *v = malloc(n * sizeof(int16_t));
    size_t got = v ? fread(v, sizeof(int16_t), n, f) : 0;
    fclose(f);
    if (got != n) { fprintf(stderr, "%s: %zu of %zu elements\n", path, got, n); exit(2); }
    return v;
}

static double now_ms(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

int main(int argc, char **argv)
{
    const int nin = (int)INFERENCE_N_INPUTS, nout = (int)INFERENCE_N_OUTPUTS;
    if (argc < 2 + nin + nout) {
        fprintf(stderr, "usage: %s WEIGHTS|- IN.bin... EXPECTED.bin... [ITERATIONS]\n", argv[0]);
        return 2;
    }
    const int iters = argc > 2 + nin + nout ? atoi(argv[2 + nin + nout]) : 1;
    int rc = inference_init(strcmp(argv[1], "-") ? argv[1] : NULL);
    if (rc) { fprintf(stderr, "inference_init: %d (%s)\n", rc, cm_last_error()); return 2; }
    inference_buf_t *bin[INFERENCE_N_INPUTS + 1], *bout[INFERENCE_N_OUTPUTS + 1];
    for (int i = 0; i < nin; ++i) {
        const io_t *t = &k_in[i];
        bin[i] = inference_buf_alloc(t->size);
        if (!bin[i]) { fprintf(stderr, "alloc failed\n"); return 2; }
        int16_t *raw = load(argv[2 + i], t->numel);
        Data_t *p = inference_buf_ptr(bin[i]);
        memset(p, 0, t->size * sizeof(Data_t));
        for (size_t e = 0; e < t->numel; ++e) p[pos_of(t, e)] = raw[e];
        free(raw);
    }
    for (int i = 0; i < nout; ++i) {
        bout[i] = inference_buf_alloc(k_out[i].size);
        if (!bout[i]) { fprintf(stderr, "alloc failed\n"); return 2; }
    }
"""]
        args = ", ".join([f"bin[{i}]" for i in range(len(ins))] + [f"bout[{i}]" for i in range(len(outs))])
        out += [f"    rc = inference_run({args});",
                "    if (rc) { fprintf(stderr, \"inference_run: %d (%s)\\n\", rc, cm_last_error()); return 2; }",
                "    int bad_total = 0;",
                "    for (int i = 0; i < nout; ++i) {",
                "        const io_t *t = &k_out[i];",
                "        int16_t *want = load(argv[2 + nin + i], t->numel);",
                "        const Data_t *p = inference_buf_ptr(bout[i]);",
                "        size_t bad = 0, first = 0;",
                "        for (size_t e = 0; e < t->numel; ++e)",
                "            if (p[pos_of(t, e)] != want[e] && bad++ == 0) first = e;",
                "        if (bad)",
                "            printf(\"%s: FAIL %zu of %u elements differ (first %zu: got %d want %d)\\n\", t->name,",
                "                   bad, t->numel, first, p[pos_of(t, first)], want[first]);",
                "        else",
                "            printf(\"%s: PASS %u elements bit-exact\\n\", t->name, t->numel);",
                "        bad_total += bad != 0;",
                "        free(want);",
                "    }",
                "    if (iters > 1) {",
                "        double t0 = now_ms();",
                "        for (int it = 0; it < iters; ++it)",
                f"            rc |= inference_run({args});",
                "        double dt = (now_ms() - t0) / iters;",
                "        printf(\"inference_run: %.4f ms mean over %d runs (host syncs included)\\n\", dt, iters);",
                "    }",
                "    for (int i = 0; i < nin; ++i) inference_buf_free(bin[i]);",
                "    for (int i = 0; i < nout; ++i) inference_buf_free(bout[i]);",
                "    inference_deinit();",
                "    return bad_total || rc ? 1 : 0;",
                "}", ""]
        return "\n".join(out)

    # ----------------------------------------------------------- build files
    def makefile(self) -> str:
        return f"""# Makefile -- generated for model '{self.name}': builds libinference.a and
# test_inference against libcormorant_amd.so (the counterpart of the reference's
# generated CMakeLists.txt; CMakeLists.txt beside this file does the same).
CORMORANT_ROOT ?= {self.root}
ROCM ?= /opt/rocm
CC ?= gcc
CFLAGS ?= -O2 -std=c11 -Wall -Wextra -D__HIP_PLATFORM_AMD__
HERE := $(dir $(abspath $(lastword $(MAKEFILE_LIST))))
INC := -I$(HERE)include -I$(CORMORANT_ROOT)/include -I$(ROCM)/include
LIBS := -L$(CORMORANT_ROOT)/cormorant_amd -lcormorant_amd -L$(ROCM)/lib -lamdhip64 \\
        -Wl,-rpath,$(CORMORANT_ROOT)/cormorant_amd -Wl,-rpath,$(ROCM)/lib

all: $(HERE)libinference.a $(HERE)test_inference

$(HERE)inference.o: $(HERE)src/inference.c $(HERE)include/inference.h
\t$(CC) $(CFLAGS) $(INC) -c -o $@ $<

$(HERE)libinference.a: $(HERE)inference.o
\tar rcs $@ $^

$(HERE)test_inference: $(HERE)test/test_inference.c $(HERE)libinference.a
\t$(CC) $(CFLAGS) $(INC) -o $@ $< $(HERE)libinference.a $(LIBS)

clean:
\trm -f $(HERE)inference.o $(HERE)libinference.a $(HERE)test_inference

.PHONY: all clean
"""

    def cmake(self) -> str:
        return f"""# CMakeLists.txt -- generated for model '{self.name}' (counterpart of the
# reference's generated CMakeLists.txt, inference-scheduler/src/codegen/_cmake.py).
cmake_minimum_required(VERSION 3.16)
project(inference_{c_identifier(self.name)} C)
set(CORMORANT_ROOT "{self.root}" CACHE PATH "root of the cormorant_amd tree")
set(ROCM_PATH "/opt/rocm" CACHE PATH "ROCm installation")
set(CMAKE_C_STANDARD 11)
add_compile_definitions(__HIP_PLATFORM_AMD__)
include_directories(${{CMAKE_CURRENT_SOURCE_DIR}}/include ${{CORMORANT_ROOT}}/include ${{ROCM_PATH}}/include)
find_library(CORMORANT_LIB cormorant_amd PATHS ${{CORMORANT_ROOT}}/cormorant_amd NO_DEFAULT_PATH REQUIRED)
find_library(HIP_LIB amdhip64 PATHS ${{ROCM_PATH}}/lib REQUIRED)
add_library(inference STATIC src/inference.c)
target_link_libraries(inference PUBLIC ${{CORMORANT_LIB}} ${{HIP_LIB}})
add_executable(test_inference test/test_inference.c)
target_link_libraries(test_inference PRIVATE inference)
"""

    # ------------------------------------------------------------------ write
    def files(self) -> Dict[str, Union[str, bytes]]:
        # the source first: it assigns the pool views the header and test use
        src = self.source()
        files: Dict[str, Union[str, bytes]] = {
            "include/inference.h": self.header(),
            "src/inference.c": src,
            "test/test_inference.c": self.test_program(),
            "Makefile": self.makefile(),
            "CMakeLists.txt": self.cmake(),
        }
        if not self.inline:
            files["weights.bin"] = self.plan.pool_image()[:self.weights_end].astype("<i2").tobytes()
        return files

    def write(self, out_dir: str) -> List[str]:
        written = []
        for rel, content in self.files().items():
            path = os.path.join(out_dir, rel)
            os.makedirs(os.path.dirname(path), exist_ok=True)
            with open(path, "wb" if isinstance(content, bytes) else "w") as f:
                f.write(content)
            written.append(path)
        return written


def write_project(model, out_dir: str, name: str = "model", **kw) -> List[str]:
    """Write the C project of `model` (OnnxGraph, ONNX bytes or path) into out_dir."""
    return ProjectWriter(model, name, **kw).write(out_dir)
