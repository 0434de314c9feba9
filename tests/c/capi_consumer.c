/* capi_consumer.c -- a C caller of the library through the reference's own
 * helper names: the shim INTEGRATION.md gives (inference_buf_* and run_* as
 * forwards to cm_buf_* / cm_run_*), used the way the reference's generated
 * inference.c uses them (_source.py:198-421, 475-791): one pool buffer with
 * views at element offsets, weights synced once, kernel calls in order, the
 * output synced back.  Every output is compared with the CPU oracle
 * (oracle/cm_oracle.h, linked as libcm_oracle.so) bit for bit.
 *
 * Test program only (built by tests/c/Makefile, run by tests/test_gpu_capi_c.py).
 * Exit status 0 = every case matched; prints one line per case.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cormorant_amd.h"
#include "cm_oracle.h"

/* ---- the shim of INTEGRATION.md ---------------------------------------- */
typedef cm_buf_t inference_buf_t;                     /* bench_src/inference.h:12-21 */
#define inference_buf_alloc          cm_buf_alloc
#define inference_buf_free           cm_buf_free
#define inference_buf_ptr            cm_buf_ptr        /* host mirror ("virt") */
#define inference_buf_init_view      cm_buf_init_view
#define inference_buf_sync_to_device(b)   cm_buf_sync_to_device(b)
#define inference_buf_sync_from_device(b) cm_buf_sync_from_device(b)

static void die(const char *what) {
    fprintf(stderr, "capi_consumer: %s: %s\n", what, cm_last_error());
    exit(2);
}
static void run_op(inference_buf_t *a, inference_buf_t *b, inference_buf_t *c, unsigned size,
                   unsigned op, unsigned outer, unsigned a_inc, unsigned b_inc)
{ if (cm_run_op(a, b, c, size, op, outer, a_inc, b_inc)) die("run_op"); }
static void run_matmul(inference_buf_t *a, inference_buf_t *b, inference_buf_t *c, unsigned n,
                       unsigned k, unsigned m, unsigned batch, unsigned as, unsigned bs, unsigned cs)
{ if (cm_run_matmul(a, b, c, n, k, m, batch, as, bs, cs)) die("run_matmul"); }
static void run_matmul_at(inference_buf_t *a, unsigned ao, inference_buf_t *b, unsigned bo,
                          inference_buf_t *c, unsigned co, unsigned n, unsigned k, unsigned m,
                          unsigned batch, unsigned as, unsigned bs, unsigned cs)
{ if (cm_run_matmul_at(a, ao, b, bo, c, co, n, k, m, batch, as, bs, cs)) die("run_matmul_at"); }
static void run_conv(inference_buf_t *x, inference_buf_t *w, inference_buf_t *bias,
                     inference_buf_t *y, unsigned batch, unsigned ic, unsigned ih, unsigned iw,
                     unsigned oc, unsigned oh, unsigned ow, unsigned kh, unsigned kw, unsigned sh,
                     unsigned sw, unsigned dh, unsigned dw, unsigned pt, unsigned pl, unsigned hb,
                     unsigned idw)
{ if (cm_run_conv(x, w, bias, y, batch, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, dh, dw, pt, pl,
                  hb, idw)) die("run_conv"); }
static void run_pool(inference_buf_t *x, inference_buf_t *y, unsigned batch, unsigned ch,
                     unsigned ih, unsigned iw, unsigned oh, unsigned ow, unsigned ph, unsigned pw,
                     unsigned sh, unsigned sw, unsigned pt, unsigned pl, unsigned dh, unsigned dw,
                     unsigned ptype, unsigned lpo, unsigned cip)
{ if (cm_run_pool(x, y, batch, ch, ih, iw, oh, ow, ph, pw, sh, sw, pt, pl, dh, dw, ptype, lpo,
                  cip)) die("run_pool"); }

/* ---- test data ---------------------------------------------------------- */
static uint64_t g_state = 0x243F6A8885A308D3ull;
static int16_t rnd16(void) {   /* xorshift64*, full int16 range */
    g_state ^= g_state >> 12;
    g_state ^= g_state << 25;
    g_state ^= g_state >> 27;
    return (int16_t)(uint16_t)((g_state * 0x2545F4914F6CDD1Dull) >> 40);
}
static void fill(int16_t *p, size_t n, int lim) {   /* lim = 0: full range */
    for (size_t i = 0; i < n; ++i) {
        int16_t v = rnd16();
        p[i] = lim ? (int16_t)(v % lim) : v;
    }
}
static int g_fail = 0;
static void check(const char *name, const int16_t *got, const int16_t *want, size_t n) {
    size_t bad = 0, first = 0;
    for (size_t i = 0; i < n; ++i)
        if (got[i] != want[i]) { if (!bad) first = i; ++bad; }
    if (bad) {
        printf("FAIL %s: %zu of %zu differ, first at %zu (got %d want %d)\n", name, bad, n, first,
               got[first], want[first]);
        g_fail = 1;
    } else {
        printf("ok   %s (%zu elements)\n", name, n);
    }
    fflush(stdout);
}

int main(void) {
    if (cm_buf_pool_init()) die("cm_buf_pool_init");

    /* A small "generated runtime": one pool holding weights and intermediates
     * as views at 64-byte-aligned element offsets, graph input / output apart.
     *   h0 = matmul(X[6x40], W1[40x24])         run_matmul_at into the pool
     *   h1 = h0 + b1 (bias row broadcast)        run_op outer=6, chunk stride 24
     *   h2 = relu(h1)                            run_op unary
     *   Y  = matmul(h2[6x24], W2[24x10]) rows    run_matmul_at with c stride 16 (row-strided)
     */
    enum { N = 6, K1 = 40, H = 24, O = 10, OS = 16 };
    const unsigned off_w1 = 0, off_b1 = 1024, off_w2 = 1088, off_h0 = 1408, off_h1 = 1600,
                   off_h2 = 1792;
    inference_buf_t *pool = inference_buf_alloc(2048);
    inference_buf_t *X = inference_buf_alloc(N * K1);
    inference_buf_t *Y = inference_buf_alloc(N * OS);
    if (!pool || !X || !Y) die("alloc");
    int16_t *P = inference_buf_ptr(pool);
    fill(P + off_w1, K1 * H, 600);
    fill(P + off_b1, H, 0);
    fill(P + off_w2, H * O, 600);
    fill(inference_buf_ptr(X), N * K1, 900);
    memset(inference_buf_ptr(Y), 0, N * OS * 2);
    inference_buf_sync_to_device(pool);
    inference_buf_sync_to_device(X);
    inference_buf_sync_to_device(Y);
    inference_buf_t w1, b1, h0, h1, h2, w2;
    inference_buf_init_view(&w1, pool, off_w1, K1 * H);
    inference_buf_init_view(&b1, pool, off_b1, H);
    inference_buf_init_view(&w2, pool, off_w2, H * O);
    inference_buf_init_view(&h0, pool, off_h0, N * H);
    inference_buf_init_view(&h1, pool, off_h1, N * H);
    inference_buf_init_view(&h2, pool, off_h2, N * H);
    run_matmul_at(X, 0, pool, off_w1, pool, off_h0, N, K1, H, 1, 0, 0, 0);
    run_op(&h0, &b1, &h1, H, CM_VECTOROP_ADD, N, H, 0);
    run_op(&h1, NULL, &h2, N * H, CM_VECTOROP_RELU, 1, 0, 0);
    /* Y rows at stride 16: batch = N matmuls of 1 x H x O (nodes.py:785-801) */
    run_matmul(&h2, &w2, Y, 1, H, O, N, H, 0, OS);
    inference_buf_sync_from_device(Y);
    inference_buf_sync_from_device(pool);
    {
        int16_t r0[N * H], r1[N * H], r2[N * H], ry[N * OS];
        memset(ry, 0, sizeof(ry));
        ora_matmul(inference_buf_ptr(X), P + off_w1, r0, N, K1, H, 1, 0, 0, 0);
        ora_vectorop(r0, P + off_b1, r1, H, CM_VECTOROP_ADD, N, H, 0);
        ora_vectorop(r1, NULL, r2, N * H, CM_VECTOROP_RELU, 1, 0, 0);
        ora_matmul(r2, P + off_w2, ry, 1, H, O, N, H, 0, OS);
        check("run_matmul_at into a pool view", P + off_h0, r0, N * H);
        check("run_op ADD broadcast rows", P + off_h1, r1, N * H);
        check("run_op RELU", P + off_h2, r2, N * H);
        check("run_matmul row-strided output", inference_buf_ptr(Y), ry, N * OS);
    }

    /* every VectorOP opcode, full-range values, flat */
    {
        enum { S = 3001 };
        inference_buf_t *a = inference_buf_alloc(S), *b = inference_buf_alloc(S),
                        *c = inference_buf_alloc(S);
        if (!a || !b || !c) die("alloc");
        fill(inference_buf_ptr(a), S, 0);
        fill(inference_buf_ptr(b), S, 0);
        inference_buf_sync_to_device(a);
        inference_buf_sync_to_device(b);
        static int16_t want[S];
        for (unsigned op = 0; op <= 6; ++op) {
            char name[64];
            run_op(a, b, c, S, op, 1, 0, 0);
            inference_buf_sync_from_device(c);
            ora_vectorop(inference_buf_ptr(a), inference_buf_ptr(b), want, S, op, 1, 0, 0);
            snprintf(name, sizeof(name), "run_op op %u", op);
            check(name, inference_buf_ptr(c), want, S);
        }
        inference_buf_free(a); inference_buf_free(b); inference_buf_free(c);
    }

    /* conv (standard with bias, depthwise) and pool (each type) */
    {
        enum { B = 2, C = 16, IH = 19, IW = 23, M = 24 };
        /* outputs: 17 x 13 for the strided conv (fits the depthwise output's size) */
        const unsigned oh = (IH + 2 * 1 - 2 * 2 - 1) / 1 + 1, ow = (IW + 2 * 2 - 1 * 2 - 1) / 2 + 1;
        inference_buf_t *x = inference_buf_alloc(B * C * IH * IW), *w = inference_buf_alloc(M * C * 9),
                        *bias = inference_buf_alloc(M), *y = inference_buf_alloc(B * C * IH * IW);
        if (!x || !w || !bias || !y) die("alloc");
        fill(inference_buf_ptr(x), B * C * IH * IW, 0);
        fill(inference_buf_ptr(w), M * C * 9, 0);
        fill(inference_buf_ptr(bias), M, 0);
        inference_buf_sync_to_device(x);
        inference_buf_sync_to_device(w);
        inference_buf_sync_to_device(bias);
        /* 3x3, stride (1, 2), dilation (2, 1), pads (1, 2): full-range values wrap */
        run_conv(x, w, bias, y, B, C, IH, IW, M, oh, ow, 3, 3, 1, 2, 2, 1, 1, 2, 1, 0);
        inference_buf_sync_from_device(y);
        int16_t *want = malloc((size_t)B * M * oh * ow * 2 + (size_t)B * C * IH * IW * 2);
        if (!want) die("malloc");
        ora_conv(inference_buf_ptr(x), inference_buf_ptr(w), inference_buf_ptr(bias), want, B, C,
                 IH, IW, M, oh, ow, 3, 3, 1, 2, 2, 1, 1, 2, 1, 0);
        check("run_conv 3x3 strided dilated with bias", inference_buf_ptr(y), want, B * M * oh * ow);
        /* depthwise 3x3 stride 1 pad 1, no bias */
        run_conv(x, w, NULL, y, B, C, IH, IW, C, IH, IW, 3, 3, 1, 1, 1, 1, 1, 1,
                 0, 1);
        inference_buf_sync_from_device(y);
        ora_conv(inference_buf_ptr(x), inference_buf_ptr(w), NULL, want, B, C, IH, IW, C, IH, IW,
                 3, 3, 1, 1, 1, 1, 1, 1, 0, 1);
        check("run_conv depthwise", inference_buf_ptr(y), want, B * C * IH * IW);
        static const unsigned types[][3] = {{0, 1, 0}, {1, 1, 1}, {1, 1, 0}, {2, 1, 0}, {2, 2, 0}};
        for (unsigned t = 0; t < 5; ++t) {
            const unsigned ph = 3, pw = 2, sh = 2, sw = 1, pt = 1, pl = 1;
            const unsigned poh = (IH + 2 * pt - ph) / sh + 1, pow_ = (IW + 2 * pl - pw) / sw + 1;
            char name[64];
            run_pool(x, y, B, C, IH, IW, poh, pow_, ph, pw, sh, sw, pt, pl, 1, 1, types[t][0],
                     types[t][1], types[t][2]);
            inference_buf_sync_from_device(y);
            ora_pool(inference_buf_ptr(x), want, B, C, IH, IW, poh, pow_, ph, pw, sh, sw, pt, pl, 1,
                     1, types[t][0], types[t][1], types[t][2]);
            snprintf(name, sizeof(name), "run_pool type %u lp %u cip %u", types[t][0], types[t][1],
                     types[t][2]);
            check(name, inference_buf_ptr(y), want, B * C * poh * pow_);
        }
        free(want);
        inference_buf_free(x); inference_buf_free(w); inference_buf_free(bias); inference_buf_free(y);
    }

    /* a call that does not fit its buffers is rejected before any launch */
    {
        inference_buf_t *a = inference_buf_alloc(16), *c = inference_buf_alloc(16);
        if (!a || !c) die("alloc");
        const int rc = cm_run_op(a, NULL, c, 17, CM_VECTOROP_RELU, 1, 0, 0);
        printf("%s run_op past the buffer end -> %d (%s)\n", rc == CM_ERR_RANGE ? "ok  " : "FAIL", rc,
               cm_last_error());
        if (rc != CM_ERR_RANGE) g_fail = 1;
        inference_buf_free(a); inference_buf_free(c);
    }
    inference_buf_free(pool); inference_buf_free(X); inference_buf_free(Y);
    cm_buf_pool_deinit();
    printf(g_fail ? "capi_consumer: FAILED\n" : "capi_consumer: all cases match the oracle\n");
    return g_fail;
}
