/*
 * cm_oracle.h -- CPU restatement of the four Cormorant Q8.8 kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle and the
 * CPU baseline.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it.
 *
 * Element type: int16 two's complement holding ap_fixed<16,8> (Q8.8).
 * Accumulator:  uint32 holding ap_fixed<32,16> raw bits (AP_TRN, AP_WRAP),
 *               so every += wraps modulo 2^32 exactly like the reference.
 *
 * Each function cites the reference file:line it restates.  The loops follow
 * the reference loop order (tile sizes from the CMake defaults) so that the
 * single-thread timing is the faithful C-simulation path; the *_omp variants
 * split the independent outermost loop over threads and give identical bits.
 */
#ifndef CM_ORACLE_H
#define CM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kernels/vectorop/kernel/VectorOP.cpp:140-188 */
void ora_vectorop(const int16_t *a, const int16_t *b, int16_t *c, uint32_t size,
                  uint32_t op, uint32_t outer, uint32_t a_inc, uint32_t b_inc);
void ora_vectorop_omp(const int16_t *a, const int16_t *b, int16_t *c, uint32_t size,
                      uint32_t op, uint32_t outer, uint32_t a_inc, uint32_t b_inc);

/* kernels/matmul/kernel/MatmulKernel.cpp:31-224 (tiles N=4, M=16, K=256; no kMaxK) */
void ora_matmul(const int16_t *a, const int16_t *b, int16_t *c, uint32_t n, uint32_t k,
                uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs);
void ora_matmul_omp(const int16_t *a, const int16_t *b, int16_t *c, uint32_t n, uint32_t k,
                    uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs);
/* One output row of one batch, naive order (kernels/matmul/test/TestMatmulSim.cpp:65-82):
 * used to check sampled rows of products too large to recompute whole. */
void ora_matmul_row(const int16_t *a_row, const int16_t *b, int16_t *c_row,
                    uint32_t k, uint32_t m);

/* kernels/conv/kernel/ConvKernel.cpp:46-343 (tiles M=8, IC=16; no kMaxKH/KW) */
void ora_conv(const int16_t *x, const int16_t *w, const int16_t *bias, int16_t *y,
              uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
              uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
              uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
              uint32_t pad_top, uint32_t pad_left, uint32_t has_bias, uint32_t is_dw);
void ora_conv_omp(const int16_t *x, const int16_t *w, const int16_t *bias, int16_t *y,
                  uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                  uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                  uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
                  uint32_t pad_top, uint32_t pad_left, uint32_t has_bias, uint32_t is_dw);

/* kernels/pool/kernel/PoolingKernel.cpp:37-275 (tile C=8; no kMaxPoolH/W) */
void ora_pool(const int16_t *x, int16_t *y, uint32_t batch, uint32_t ch,
              uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
              uint32_t ph, uint32_t pw, uint32_t sh, uint32_t sw,
              uint32_t pad_top, uint32_t pad_left, uint32_t dh, uint32_t dw,
              uint32_t pool_type, uint32_t lp_order, uint32_t cip);
void ora_pool_omp(const int16_t *x, int16_t *y, uint32_t batch, uint32_t ch,
                  uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
                  uint32_t ph, uint32_t pw, uint32_t sh, uint32_t sw,
                  uint32_t pad_top, uint32_t pad_left, uint32_t dh, uint32_t dw,
                  uint32_t pool_type, uint32_t lp_order, uint32_t cip);

/* Scalar finalisers, exported so tests can sweep them exhaustively. */
int16_t ora_q88_mul(int16_t a, int16_t b);
int16_t ora_q88_div(int16_t a, int16_t b);
int16_t ora_avg_finalize(uint32_t acc, uint32_t denom);   /* PoolingKernel.cpp:137, 259, 265 */
int16_t ora_lp2_finalize(uint32_t acc);                   /* PoolingKernel.cpp:263, 265 */
/* Sum over a in [lo, hi) of (uint16)ora_lp2_finalize(a) * (a | 1), modulo 2^64. */
uint64_t ora_lp2_checksum(uint32_t lo, uint32_t hi);
/* Sum over v in [lo, lo+count) of (uint16)ora_avg_finalize(v << 8, denom) * (v | 1). */
uint64_t ora_avg_checksum(uint32_t lo, uint32_t count, uint32_t denom);

void ora_set_threads(int n);
int ora_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
