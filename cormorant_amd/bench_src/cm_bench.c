/* cm_bench.c -- per-case latency / throughput benchmark of the four kernels on
 * one MI355X, the counterpart of the reference's KV260 benchmark programs
 * (inference-scheduler/bench_src/bench_vectorop.c, bench_matmul.c,
 * bench_conv.c, bench_pool.c).  Same arguments, same timing loop (one call,
 * then sync_from_device of the output, `iters` times after `warmup` calls),
 * same metric formulas and JSON fields, through the same buffer-level API
 * (cm_buf_* / cm_run_*, the counterparts of inference_buf_* / run_*).
 *
 * Usage, one case per invocation (arguments as the reference's programs):
 *   cm_bench vectorop instance label op size outer a_inc b_inc iters [warmup]
 *   cm_bench matmul   instance label n k m batch a_stride b_stride iters [warmup]
 *   cm_bench conv     instance label batch in_ch in_h in_w out_ch kh kw sh sw
 *                                    dh dw pt pl has_bias is_dw iters [warmup]
 *   cm_bench pool     instance label batch channels in_h in_w pool_h pool_w sh sw
 *                                    pt pl dh dw pool_type lp_order cip iters [warmup]
 * or many cases, one such argument line per input line (without "cm_bench"):
 *   cm_bench -  < cases.txt
 * `instance` is the GPU ordinal (the reference's UIO device name; a
 * non-numeric value means device 0).
 *
 * Output: one JSON line per case with the reference's fields, where lat_ms and
 * gbs / gops follow the reference's loop (call + sync_from_device, i.e. the
 * output copied back to the host each iteration), plus
 *   kernel_ms, gbs_kernel / gops_kernel: device time per call, HIP events
 *       around `iters` back-to-back calls on the stream (no host copy);
 *   seed, out_fnv1a: the inputs are filled from splitmix64(seed + buffer index)
 *       (low 16 bits per element) instead of the reference's memset(1), and
 *       the FNV-1a 64 hash of the output's bytes identifies the result; with
 *       CM_BENCH_DUMP=<dir> the output is also written raw (int16, little
 *       endian) to <dir>/<label>.bin, so a checker can recompute the case on
 *       the CPU and compare element by element.
 * Split-K scratch is a caller-owned workspace (cm_buf_alloc, sized by
 * cm_*_workspace_size) set with cm_set_workspace, as a generated runtime would.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "cormorant_amd.h"

#define MAX_ARGS 24

static uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* element i of buffer `which`: low 16 bits of splitmix64(seed_i), where the
 * counter runs seed_i = base + i * golden (the generator's own increment) */
static void fill(cm_buf_t *b, uint64_t seed, uint32_t which) {
    int16_t *h = cm_buf_ptr(b);
    const uint64_t base = seed * 0x100000001B3ull + which;
    for (uint32_t i = 0; i < cm_buf_count(b); ++i)
        h[i] = (int16_t)(uint16_t)splitmix64(base + (uint64_t)i * 0x9E3779B97F4A7C15ull);
}

static uint64_t fnv1a(const int16_t *p, uint32_t n) {
    const uint8_t *b = (const uint8_t *)p;
    uint64_t h = 0xCBF29CE484222325ull;
    for (uint64_t i = 0; i < 2ull * n; ++i) {
        h ^= b[i];
        h *= 0x100000001B3ull;
    }
    return h;
}

static double now_ms(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec * 1e3 + (double)t.tv_nsec * 1e-6;
}

static unsigned u(const char *s) { return (unsigned)strtoul(s, NULL, 0); }

/* One case: the argument values, the buffers, and the call. */
typedef struct bench_case {
    int kind;   /* 0 vectorop, 1 matmul, 2 conv, 3 pool */
    const char *label;
    unsigned v[20];
    cm_buf_t *buf[4];
    cm_buf_t *out;
} bench_case_t;

static int run_once(const bench_case_t *c) {
    const unsigned *v = c->v;
    cm_buf_t *const *b = c->buf;
    switch (c->kind) {
    case 0: return cm_run_op(b[0], b[1], b[2], v[1], v[0], v[2], v[3], v[4]);
    case 1: return cm_run_matmul(b[0], b[1], b[2], v[0], v[1], v[2], v[3], v[4], v[5], v[0] * v[2]);
    case 2: return cm_run_conv(b[0], b[1], b[2], b[3], v[0], v[1], v[2], v[3], v[4], v[15], v[16],
                               v[5], v[6], v[7], v[8], v[9], v[10], v[11], v[12], v[13], v[14]);
    default: return cm_run_pool(b[0], b[1], v[0], v[1], v[2], v[3], v[15], v[16], v[4], v[5],
                                v[6], v[7], v[8], v[9], v[10], v[11], v[12], v[13], v[14]);
    }
}

static int fail(const char *what, int rc) {
    fprintf(stderr, "cm_bench: %s failed (%d): %s\n", what, rc, cm_last_error());
    return 1;
}

/* argv: kind instance label values... iters [warmup] */
static int bench(int argc, char **argv, uint64_t seed) {
    static const char *kinds[] = {"vectorop", "matmul", "conv", "pool"};
    static const int nvals[] = {5, 6, 15, 15};
    bench_case_t c;
    memset(&c, 0, sizeof(c));
    c.kind = -1;
    for (int k = 0; k < 4; ++k)
        if (argc > 0 && strcmp(argv[0], kinds[k]) == 0) c.kind = k;
    if (c.kind < 0 || argc < 4 + nvals[c.kind]) {
        fprintf(stderr, "cm_bench: expected '<vectorop|matmul|conv|pool> instance label <%s args> "
                        "iters [warmup]'\n", c.kind < 0 ? "kernel" : kinds[c.kind]);
        return 1;
    }
    const int nv = nvals[c.kind];
    char *end = NULL;
    const long dev = strtol(argv[1], &end, 0);
    if (end && *end == '\0' && dev >= 0) {
        const hipError_t e = hipSetDevice((int)dev);
        if (e != hipSuccess) { fprintf(stderr, "cm_bench: no GPU %ld\n", dev); return 1; }
    }
    c.label = argv[2];
    for (int i = 0; i < nv; ++i) c.v[i] = u(argv[3 + i]);
    const unsigned iters = u(argv[3 + nv]);
    const unsigned warmup = argc > 4 + nv ? u(argv[4 + nv]) : 10u;
    unsigned *v = c.v;

    /* buffer sizes as the reference programs allocate them */
    uint32_t n_elem[4] = {0, 0, 0, 0};
    int nbuf = 0;
    size_t ws = 0;
    double bytes = 0, ops = 0;
    if (c.kind == 0) {   /* op size outer a_inc b_inc (bench_vectorop.c:55-58, 93-95) */
        const unsigned op = v[0], sz = v[1], outer = v[2], ai = v[3], bi = v[4];
        n_elem[0] = ai ? outer * sz : sz;
        n_elem[1] = bi ? outer * sz : sz;
        n_elem[2] = outer * sz;
        nbuf = 3;
        bytes = (double)(op >= 4u ? 2u : 3u) * n_elem[2] * 2.0;
    } else if (c.kind == 1) {   /* n k m batch as bs (bench_matmul.c:62-64, 95) */
        const unsigned n = v[0], kd = v[1], m = v[2], batch = v[3], as = v[4], bs = v[5];
        n_elem[0] = as ? batch * n * kd : n * kd;
        n_elem[1] = bs ? batch * kd * m : kd * m;
        n_elem[2] = batch * n * m;
        nbuf = 3;
        ops = 2.0 * n * kd * m * batch;
        ws = cm_matmul_workspace_size(n, kd, m, batch, as, bs, n * m);
    } else if (c.kind == 2) {   /* bench_conv.c:74-75, 85-88, 127-132 */
        const unsigned batch = v[0], ic = v[1], ih = v[2], iw = v[3], oc = v[4], kh = v[5],
                       kw = v[6], sh = v[7], sw = v[8], dh = v[9], dw = v[10], pt = v[11],
                       pl = v[12], hb = v[13], idw = v[14];
        const unsigned oh = (ih + 2 * pt - dh * (kh - 1) - 1) / sh + 1;
        const unsigned ow = (iw + 2 * pl - dw * (kw - 1) - 1) / sw + 1;
        v[15] = oh;
        v[16] = ow;
        n_elem[0] = batch * ic * ih * iw;
        n_elem[1] = idw ? oc * kh * kw : oc * ic * kh * kw;
        n_elem[2] = hb ? oc : 1u;
        n_elem[3] = batch * oc * oh * ow;
        nbuf = 4;
        ops = 2.0 * batch * oc * oh * ow * (idw ? (double)kh * kw : (double)ic * kh * kw);
        ws = cm_conv_workspace_size(batch, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl,
                                    hb, idw);
    } else {   /* bench_pool.c:71-72, 82-83, 116-117 */
        const unsigned batch = v[0], ch = v[1], ih = v[2], iw = v[3], ph = v[4], pw = v[5],
                       sh = v[6], sw = v[7], pt = v[8], pl = v[9], dh = v[10], dw = v[11];
        const unsigned oh = (ih + 2 * pt - dh * (ph - 1) - 1) / sh + 1;
        const unsigned ow = (iw + 2 * pl - dw * (pw - 1) - 1) / sw + 1;
        v[15] = oh;
        v[16] = ow;
        n_elem[0] = batch * ch * ih * iw;
        n_elem[1] = batch * ch * oh * ow;
        nbuf = 2;
        bytes = ((double)n_elem[0] + n_elem[1]) * 2.0;
    }
    int rc = cm_buf_pool_init();
    if (rc) return fail("cm_buf_pool_init", rc);
    for (int i = 0; i < nbuf; ++i) {
        c.buf[i] = cm_buf_alloc(n_elem[i]);
        if (!c.buf[i]) return fail("cm_buf_alloc", CM_ERR_NOMEM);
        fill(c.buf[i], seed, (uint32_t)i);
        if ((rc = cm_buf_sync_to_device(c.buf[i]))) return fail("sync_to_device", rc);
    }
    c.out = c.buf[nbuf - 1];
    cm_buf_t *wsb = NULL;
    if (ws) {   /* caller-owned split-K workspace, as in a generated runtime's pool */
        wsb = cm_buf_alloc((uint32_t)((ws + 1) / 2));
        if (!wsb) return fail("cm_buf_alloc(workspace)", CM_ERR_NOMEM);
        cm_set_workspace(cm_buf_dev(wsb), ws);
    }

    for (unsigned i = 0; i < warmup; ++i) {
        if ((rc = run_once(&c))) return fail(c.label, rc);
        if ((rc = cm_buf_sync_from_device(c.out))) return fail("sync_from_device", rc);
    }
    /* the reference's loop: call, then sync_from_device of the output */
    const double t0 = now_ms();
    for (unsigned i = 0; i < iters; ++i) {
        if ((rc = run_once(&c))) return fail(c.label, rc);
        if ((rc = cm_buf_sync_from_device(c.out))) return fail("sync_from_device", rc);
    }
    const double lat = (now_ms() - t0) / (double)(iters ? iters : 1);
    /* device time: HIP events on the library stream around back-to-back calls */
    hipEvent_t e0, e1;
    float kms = 0.f;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
        return fail("hipEventCreate", CM_ERR_HIP);
    hipEventRecord(e0, cm_get_stream());
    for (unsigned i = 0; i < iters; ++i)
        if ((rc = run_once(&c))) return fail(c.label, rc);
    hipEventRecord(e1, cm_get_stream());
    if (hipEventSynchronize(e1) != hipSuccess) return fail("hipEventSynchronize", CM_ERR_HIP);
    hipEventElapsedTime(&kms, e0, e1);
    const double kernel_ms = (double)kms / (double)(iters ? iters : 1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if ((rc = cm_buf_sync_from_device(c.out))) return fail("sync_from_device", rc);
    const uint64_t h = fnv1a(cm_buf_ptr(c.out), cm_buf_count(c.out));
    const char *dump = getenv("CM_BENCH_DUMP");
    if (dump && dump[0]) {
        char path[1024];
        snprintf(path, sizeof(path), "%s/%s.bin", dump, c.label);
        FILE *f = fopen(path, "wb");
        if (!f || fwrite(cm_buf_ptr(c.out), 2, cm_buf_count(c.out), f) != cm_buf_count(c.out)) {
            if (f) fclose(f);
            fprintf(stderr, "cm_bench: cannot write %s\n", path);
            return 1;
        }
        fclose(f);
    }

    switch (c.kind) {
    case 0:
        printf("{\"kernel\":\"VectorOPKernel\",\"label\":\"%s\",\"op\":%u,\"size\":%u,\"outer\":%u,"
               "\"a_inc\":%u,\"b_inc\":%u,\"iters\":%u,\"lat_ms\":%.4f,\"gbs\":%.3f",
               c.label, v[0], v[1], v[2], v[3], v[4], iters, lat, bytes / (lat * 1e-3) / 1e9);
        printf(",\"kernel_ms\":%.5f,\"gbs_kernel\":%.3f", kernel_ms, bytes / (kernel_ms * 1e-3) / 1e9);
        break;
    case 1:
        printf("{\"kernel\":\"MatmulKernel\",\"label\":\"%s\",\"n\":%u,\"k\":%u,\"m\":%u,\"batch\":%u,"
               "\"a_str\":%u,\"b_str\":%u,\"iters\":%u,\"lat_ms\":%.4f,\"gops\":%.4f",
               c.label, v[0], v[1], v[2], v[3], v[4], v[5], iters, lat, ops / (lat * 1e-3) / 1e9);
        printf(",\"kernel_ms\":%.5f,\"gops_kernel\":%.3f", kernel_ms, ops / (kernel_ms * 1e-3) / 1e9);
        break;
    case 2:
        printf("{\"kernel\":\"ConvKernel\",\"label\":\"%s\",\"batch\":%u,\"in_ch\":%u,\"in_h\":%u,"
               "\"in_w\":%u,\"out_ch\":%u,\"out_h\":%u,\"out_w\":%u,\"kh\":%u,\"kw\":%u,\"sh\":%u,"
               "\"sw\":%u,\"is_dw\":%u,\"iters\":%u,\"lat_ms\":%.4f,\"gops\":%.4f",
               c.label, v[0], v[1], v[2], v[3], v[4], v[15], v[16], v[5], v[6], v[7], v[8], v[14],
               iters, lat, ops / (lat * 1e-3) / 1e9);
        printf(",\"kernel_ms\":%.5f,\"gops_kernel\":%.3f", kernel_ms, ops / (kernel_ms * 1e-3) / 1e9);
        break;
    default:
        printf("{\"kernel\":\"PoolingKernel\",\"label\":\"%s\",\"batch\":%u,\"channels\":%u,"
               "\"in_h\":%u,\"in_w\":%u,\"out_h\":%u,\"out_w\":%u,\"pool_h\":%u,\"pool_w\":%u,"
               "\"pool_type\":%u,\"iters\":%u,\"lat_ms\":%.4f,\"gbs\":%.3f",
               c.label, v[0], v[1], v[2], v[3], v[15], v[16], v[4], v[5], v[12], iters, lat,
               bytes / (lat * 1e-3) / 1e9);
        printf(",\"kernel_ms\":%.5f,\"gbs_kernel\":%.3f", kernel_ms, bytes / (kernel_ms * 1e-3) / 1e9);
        break;
    }
    printf(",\"workspace_bytes\":%zu,\"seed\":%llu,\"out_fnv1a\":\"%016llx\"}\n", ws,
           (unsigned long long)seed, (unsigned long long)h);
    fflush(stdout);
    cm_set_workspace(NULL, 0);
    if (wsb) cm_buf_free(wsb);
    for (int i = 0; i < nbuf; ++i) cm_buf_free(c.buf[i]);
    return 0;
}

int main(int argc, char **argv) {
    const char *s = getenv("CM_BENCH_SEED");
    const uint64_t seed = s ? strtoull(s, NULL, 0) : 42u;
    if (argc >= 2 && strcmp(argv[1], "-") == 0) {   /* one case per stdin line */
        char line[1024];
        int status = 0;
        while (fgets(line, sizeof(line), stdin)) {
            char *av[MAX_ARGS];
            int ac = 0;
            for (char *t = strtok(line, " \t\r\n"); t && ac < MAX_ARGS; t = strtok(NULL, " \t\r\n"))
                av[ac++] = t;
            if (ac == 0 || av[0][0] == '#') continue;
            if (bench(ac, av, seed)) status = 1;
        }
        return status;
    }
    return bench(argc - 1, argv + 1, seed);
}
