/*
 * cm_oracle.c -- CPU restatement of Cormorant's VectorOPKernel, MatmulKernel,
 * ConvKernel and PoolingKernel with ap_fixed<16,8> data and ap_fixed<32,16>
 * accumulators, written as plain C integer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle + CPU baseline).  The product
 * library never links or calls this file.
 *
 * Type model (the Xilinx ap_fixed header is not vendored in the reference; its
 * published semantics are restated here):
 *   Data_t    = ap_fixed<16,8>   -> int16 raw r, value r/256.
 *   AccData_t = ap_fixed<32,16>  -> raw bits held in uint32, value raw/65536,
 *               AP_TRN quantisation + AP_WRAP overflow, so "+=" is addition
 *               modulo 2^32 and Data_t -> AccData_t is raw << 8.
 *   Data_t * Data_t is exact (16 fractional bits): raw product a*b in 2^-16.
 *   saturate_cast<Data_t>(acc)  (kernels/vectorop/include/VectorOP.h:30-39)
 *               = AP_TRN (floor, arithmetic >> 8) then AP_SAT clamp.
 *   (float)acc  = acc/65536 rounded to nearest even (exact power-of-two scale).
 *   AccData_t(float f) = floor(f * 65536) wrapped modulo 2^32 (AP_TRN, AP_WRAP);
 *               NaN/Inf are unpinned by any reference test and map to 0 here.
 */
#include "cm_oracle.h"

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Tile sizes from the reference CMake defaults. */
enum { MM_TILE_N = 4, MM_TILE_M = 16, MM_TILE_K = 256 };  /* kernels/matmul/CMakeLists.txt:50-57 */
enum { CV_TILE_M = 8, CV_TILE_IC = 16 };                  /* kernels/conv/CMakeLists.txt:49-56 */
enum { PL_TILE_C = 8 };                                   /* kernels/pool/CMakeLists.txt:54-55 */

static inline int16_t sat16(int64_t v) {
    return (int16_t)(v > 32767 ? 32767 : (v < -32768 ? -32768 : v));
}

/* saturate_cast<ap_fixed<16,8>>(ap_fixed<32,16> acc): floor to 8 fractional
 * bits (arithmetic shift) then clamp.  VectorOP.h:30-39, MatmulKernel.h:26-32. */
static inline int16_t acc_to_data(uint32_t acc) {
    int32_t s = (int32_t)acc;
    return sat16(s >> 8);
}

static inline uint32_t data_to_acc(int16_t x) { return (uint32_t)(int32_t)x << 8; }

/* (float) of an ap_fixed<32,16>: round-to-nearest-even of raw/65536. */
static inline float acc_to_float(uint32_t acc) {
    return (float)(int32_t)acc * (1.0f / 65536.0f);
}

/* AccData_t(float): floor to 2^-16 and wrap modulo 2^32. */
static inline uint32_t float_to_acc(float f) {
    if (!isfinite(f)) return 0u;
    double s = floor((double)f * 65536.0);
    if (s >= 9.2e18 || s <= -9.2e18) return 0u;
    return (uint32_t)(uint64_t)(int64_t)s;
}

/* ------------------------------------------------------------------------ */
/* VectorOP: kernels/vectorop/kernel/VectorOP.cpp:8-35 (scalar helpers)      */
/* ------------------------------------------------------------------------ */

/* sub_mul: ap_fixed<32,16> product, saturate_cast floors 8 bits. */
int16_t ora_q88_mul(int16_t a, int16_t b) {
    int32_t p = (int32_t)a * (int32_t)b;
    return sat16(p >> 8);
}

/* sub_div: b == 0 -> 0; quotient keeps 8 fractional bits with C integer
 * division (truncation toward zero) of a_raw * 2^8 by b_raw, then saturates
 * (VectorOP.cpp:22-25; doc/SIMULATION_ISSUES.md:226). */
int16_t ora_q88_div(int16_t a, int16_t b) {
    if (b == 0) return 0;
    int32_t q = ((int32_t)a * 256) / (int32_t)b;
    return sat16(q);
}

static inline int16_t vec_op(uint32_t op, int16_t a, int16_t b) {
    switch (op) {
    case 0: return sat16((int32_t)a + (int32_t)b);           /* OP_ADD  VectorOP.cpp:8-10  */
    case 1: return sat16((int32_t)a - (int32_t)b);           /* OP_SUB  VectorOP.cpp:12-14 */
    case 2: return ora_q88_mul(a, b);                        /* OP_MUL  VectorOP.cpp:17-19 */
    case 3: return ora_q88_div(a, b);                        /* OP_DIV  VectorOP.cpp:22-25 */
    case 4: return a < 0 ? 0 : a;                            /* OP_RELU VectorOP.cpp:27-29 */
    case 5: return a < 0 ? 0 : (a > 1536 ? 1536 : a);        /* OP_RELU6 VectorOP.cpp:31-35 */
    default: return a;                                       /* copy    VectorOP.cpp:112   */
    }
}

/* Top function VectorOP.cpp:140-188: c[o*(a_inc+b_inc)+i] = op(a[o*a_inc+i],
 * b[o*b_inc+i]); b is not read for op >= 4 (load_b feeds zeros, :68-86).  The
 * outer loop runs in order, so overlapping writes keep the last outer step. */
void ora_vectorop(const int16_t *a, const int16_t *b, int16_t *c, uint32_t size,
                  uint32_t op, uint32_t outer, uint32_t a_inc, uint32_t b_inc) {
    const uint64_t c_inc = (uint64_t)a_inc + b_inc;
    for (uint32_t o = 0; o < outer; ++o) {
        const int16_t *ap = a + (uint64_t)o * a_inc;
        const int16_t *bp = (op < 4) ? b + (uint64_t)o * b_inc : NULL;
        int16_t *cp = c + (uint64_t)o * c_inc;
        for (uint32_t i = 0; i < size; ++i)
            cp[i] = vec_op(op, ap[i], bp ? bp[i] : (int16_t)0);
    }
}

void ora_vectorop_omp(const int16_t *a, const int16_t *b, int16_t *c, uint32_t size,
                      uint32_t op, uint32_t outer, uint32_t a_inc, uint32_t b_inc) {
    const uint64_t c_inc = (uint64_t)a_inc + b_inc;
    if (outer > 1 && c_inc < size) {   /* overlapping outputs: keep sequential order */
        ora_vectorop(a, b, c, size, op, outer, a_inc, b_inc);
        return;
    }
    for (uint32_t o = 0; o < outer; ++o) {
        const int16_t *ap = a + (uint64_t)o * a_inc;
        const int16_t *bp = (op < 4) ? b + (uint64_t)o * b_inc : NULL;
        int16_t *cp = c + (uint64_t)o * c_inc;
        int64_t n = size;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i)
            cp[i] = vec_op(op, ap[i], bp ? bp[i] : (int16_t)0);
    }
}

/* ------------------------------------------------------------------------ */
/* MatMul: kernels/matmul/kernel/MatmulKernel.cpp:31-224                      */
/* ------------------------------------------------------------------------ */

/* One (batch, n_tile) unit of the reference loop nest: MatmulKernel.cpp:119-222. */
static void matmul_ntile(const int16_t *a_ptr, const int16_t *b_ptr, int16_t *c_ptr,
                         uint32_t n, uint32_t k, uint32_t m, uint32_t n_off) {
    const uint32_t n_valid = (n - n_off) < MM_TILE_N ? (n - n_off) : MM_TILE_N;
    const uint32_t m_tiles = (m + MM_TILE_M - 1) / MM_TILE_M;
    const uint32_t k_tiles = (k + MM_TILE_K - 1) / MM_TILE_K;
    for (uint32_t mt = 0; mt < m_tiles; ++mt) {
        const uint32_t m_off = mt * MM_TILE_M;
        const uint32_t m_valid = (m - m_off) < MM_TILE_M ? (m - m_off) : MM_TILE_M;
        uint32_t acc[MM_TILE_N][MM_TILE_M] = {{0}};              /* :154-161 */
        for (uint32_t kt = 0; kt < k_tiles; ++kt) {
            const uint32_t k_off = kt * MM_TILE_K;
            const uint32_t k_valid = (k - k_off) < MM_TILE_K ? (k - k_off) : MM_TILE_K;
            /* ki loop :196-205 with n1 = ki % TILE_N, kk = ki / TILE_N */
            for (uint32_t kk = 0; kk < k_valid; ++kk) {
                for (uint32_t n1 = 0; n1 < n_valid; ++n1) {
                    const int32_t av = a_ptr[(uint64_t)(n_off + n1) * k + k_off + kk];
                    const int16_t *brow = b_ptr + (uint64_t)(k_off + kk) * m + m_off;
                    for (uint32_t m1 = 0; m1 < m_valid; ++m1)
                        acc[n1][m1] += (uint32_t)(av * (int32_t)brow[m1]);
                }
            }
        }
        for (uint32_t n1 = 0; n1 < n_valid; ++n1)                /* :212-220 */
            for (uint32_t m1 = 0; m1 < m_valid; ++m1)
                c_ptr[(uint64_t)(n_off + n1) * m + m_off + m1] = acc_to_data(acc[n1][m1]);
    }
}

void ora_matmul(const int16_t *a, const int16_t *b, int16_t *c, uint32_t n, uint32_t k,
                uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs) {
    const uint32_t n_tiles = (n + MM_TILE_N - 1) / MM_TILE_N;
    for (uint32_t bi = 0; bi < batch; ++bi)                        /* :108 */
        for (uint32_t nt = 0; nt < n_tiles; ++nt)
            matmul_ntile(a + (uint64_t)bi * a_bs, b + (uint64_t)bi * b_bs,
                         c + (uint64_t)bi * c_bs, n, k, m, nt * MM_TILE_N);
}

void ora_matmul_omp(const int16_t *a, const int16_t *b, int16_t *c, uint32_t n, uint32_t k,
                    uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs) {
    const int64_t n_tiles = (n + MM_TILE_N - 1) / MM_TILE_N;
    const int64_t units = (int64_t)batch * n_tiles;
    if (batch > 1 && (uint64_t)c_bs < (uint64_t)n * m) {
        /* batch outputs overlap (c_bs = 0: every batch writes the same C): the
         * sequential batch order decides each shared element */
        ora_matmul(a, b, c, n, k, m, batch, a_bs, b_bs, c_bs);
        return;
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t u = 0; u < units; ++u) {
        const uint32_t bi = (uint32_t)(u / n_tiles), nt = (uint32_t)(u % n_tiles);
        matmul_ntile(a + (uint64_t)bi * a_bs, b + (uint64_t)bi * b_bs,
                     c + (uint64_t)bi * c_bs, n, k, m, nt * MM_TILE_N);
    }
}

void ora_matmul_row(const int16_t *a_row, const int16_t *b, int16_t *c_row,
                    uint32_t k, uint32_t m) {
    for (uint32_t j = 0; j < m; ++j) {
        uint32_t acc = 0;
        for (uint32_t kk = 0; kk < k; ++kk)
            acc += (uint32_t)((int32_t)a_row[kk] * (int32_t)b[(uint64_t)kk * m + j]);
        c_row[j] = acc_to_data(acc);
    }
}

/* ------------------------------------------------------------------------ */
/* Conv: kernels/conv/kernel/ConvKernel.cpp:46-343                            */
/* ------------------------------------------------------------------------ */

static void conv_row(const int16_t *x, const int16_t *w, const int16_t *bias, int16_t *y,
                     uint32_t ni, uint32_t oh, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                     uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                     uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
                     uint32_t pad_top, uint32_t pad_left, uint32_t has_bias, uint32_t is_dw) {
    const uint32_t m_tiles = (out_ch + CV_TILE_M - 1) / CV_TILE_M;
    const uint32_t ic_tiles = (in_ch + CV_TILE_IC - 1) / CV_TILE_IC;
    const uint64_t hw = (uint64_t)in_h * in_w;
    const uint64_t ohw = (uint64_t)out_h * out_w;
    for (uint32_t ow = 0; ow < out_w; ++ow) {
        for (uint32_t mt = 0; mt < m_tiles; ++mt) {
            const uint32_t m_off = mt * CV_TILE_M;
            const uint32_t m_valid = (out_ch - m_off) < CV_TILE_M ? (out_ch - m_off) : CV_TILE_M;
            uint32_t acc[CV_TILE_M] = {0};                          /* :160-163 */
            if (has_bias)                                           /* :164-169 */
                for (uint32_t m1 = 0; m1 < m_valid; ++m1) acc[m1] = data_to_acc(bias[m_off + m1]);
            if (!is_dw) {
                /* standard path :171-249: patch of ic_valid x kh x kw, zero outside */
                for (uint32_t ict = 0; ict < ic_tiles; ++ict) {
                    const uint32_t ic_off = ict * CV_TILE_IC;
                    const uint32_t ic_valid = (in_ch - ic_off) < CV_TILE_IC ? (in_ch - ic_off) : CV_TILE_IC;
                    for (uint32_t ic = 0; ic < ic_valid; ++ic) {
                        const int16_t *xc = x + ((uint64_t)ni * in_ch + ic_off + ic) * hw;
                        for (uint32_t khi = 0; khi < kh; ++khi) {
                            const int64_t ih = (int64_t)oh * sh + (int64_t)khi * dh - pad_top;
                            const int ih_ok = ih >= 0 && ih < (int64_t)in_h;
                            for (uint32_t kwi = 0; kwi < kw; ++kwi) {
                                const int64_t iw = (int64_t)ow * sw + (int64_t)kwi * dw - pad_left;
                                const int32_t xv = (ih_ok && iw >= 0 && iw < (int64_t)in_w)
                                                       ? xc[(uint64_t)ih * in_w + (uint64_t)iw] : 0;
                                for (uint32_t m1 = 0; m1 < m_valid; ++m1) {
                                    const int32_t wv = w[(((uint64_t)(m_off + m1) * in_ch + ic_off + ic) * kh + khi) * kw + kwi];
                                    acc[m1] += (uint32_t)(xv * wv);   /* :235-237 */
                                }
                            }
                        }
                    }
                }
            } else {
                /* depthwise path :251-319: lane m reads input channel m */
                for (uint32_t m1 = 0; m1 < m_valid; ++m1) {
                    const int16_t *xc = x + ((uint64_t)ni * in_ch + m_off + m1) * hw;
                    for (uint32_t khi = 0; khi < kh; ++khi) {
                        const int64_t ih = (int64_t)oh * sh + (int64_t)khi * dh - pad_top;
                        const int ih_ok = ih >= 0 && ih < (int64_t)in_h;
                        for (uint32_t kwi = 0; kwi < kw; ++kwi) {
                            const int64_t iw = (int64_t)ow * sw + (int64_t)kwi * dw - pad_left;
                            const int32_t xv = (ih_ok && iw >= 0 && iw < (int64_t)in_w)
                                                   ? xc[(uint64_t)ih * in_w + (uint64_t)iw] : 0;
                            const int32_t wv = w[((uint64_t)(m_off + m1) * kh + khi) * kw + kwi];
                            acc[m1] += (uint32_t)(xv * wv);          /* :308-310 */
                        }
                    }
                }
            }
            uint64_t y_addr = ((uint64_t)ni * out_ch + m_off) * ohw + (uint64_t)oh * out_w + ow;
            for (uint32_t m1 = 0; m1 < m_valid; ++m1) {              /* :329-335 */
                y[y_addr] = acc_to_data(acc[m1]);
                y_addr += ohw;
            }
        }
    }
}

void ora_conv(const int16_t *x, const int16_t *w, const int16_t *bias, int16_t *y,
              uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
              uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
              uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
              uint32_t pad_top, uint32_t pad_left, uint32_t has_bias, uint32_t is_dw) {
    for (uint32_t ni = 0; ni < batch; ++ni)                         /* :142 */
        for (uint32_t oh = 0; oh < out_h; ++oh)
            conv_row(x, w, bias, y, ni, oh, in_ch, in_h, in_w, out_ch, out_h, out_w,
                     kh, kw, sh, sw, dh, dw, pad_top, pad_left, has_bias, is_dw);
}

void ora_conv_omp(const int16_t *x, const int16_t *w, const int16_t *bias, int16_t *y,
                  uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                  uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                  uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
                  uint32_t pad_top, uint32_t pad_left, uint32_t has_bias, uint32_t is_dw) {
    const int64_t units = (int64_t)batch * out_h;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t u = 0; u < units; ++u)
        conv_row(x, w, bias, y, (uint32_t)(u / out_h), (uint32_t)(u % out_h), in_ch, in_h,
                 in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left,
                 has_bias, is_dw);
}

/* ------------------------------------------------------------------------ */
/* Pool: kernels/pool/kernel/PoolingKernel.cpp:37-275                         */
/* ------------------------------------------------------------------------ */

/* AVG finaliser: inv_denom = denom ? 1.0f/(float)denom : 0 (:134-137);
 * result = AccData_t((float)acc * inv_denom) (:259); saturate_cast (:265). */
int16_t ora_avg_finalize(uint32_t acc, uint32_t denom) {
    const float inv = denom > 0u ? 1.0f / (float)denom : 0.0f;
    const float f = acc_to_float(acc) * inv;
    return acc_to_data(float_to_acc(f));
}

/* LP p=2 finaliser: AccData_t(sqrtf((float)acc)) (:263), saturate_cast (:265).
 * A wrapped (negative) accumulator gives NaN, which maps to 0 (unpinned). */
int16_t ora_lp2_finalize(uint32_t acc) {
    const float f = sqrtf(acc_to_float(acc));
    return acc_to_data(float_to_acc(f));
}

uint64_t ora_lp2_checksum(uint32_t lo, uint32_t hi) {
    uint64_t s = 0;
#pragma omp parallel for reduction(+ : s) schedule(static)
    for (int64_t a = lo; a < (int64_t)hi; ++a)
        s += (uint64_t)(uint16_t)ora_lp2_finalize((uint32_t)a) * ((uint64_t)a | 1u);
    return s;
}

uint64_t ora_avg_checksum(uint32_t lo, uint32_t count, uint32_t denom) {
    uint64_t s = 0;
#pragma omp parallel for reduction(+ : s) schedule(static)
    for (int64_t i = 0; i < (int64_t)count; ++i) {
        const uint32_t v = lo + (uint32_t)i;
        s += (uint64_t)(uint16_t)ora_avg_finalize(v << 8, denom) * ((uint64_t)v | 1u);
    }
    return s;
}

static void pool_row(const int16_t *x, int16_t *y, uint32_t ni, uint32_t oh, uint32_t ch,
                     uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
                     uint32_t ph, uint32_t pw, uint32_t sh, uint32_t sw,
                     uint32_t pad_top, uint32_t pad_left, uint32_t dh, uint32_t dw,
                     uint32_t pool_type, uint32_t lp_order, uint32_t cip) {
    const uint32_t c_tiles = (ch + PL_TILE_C - 1) / PL_TILE_C;
    const uint64_t hw = (uint64_t)in_h * in_w;
    const uint64_t ohw = (uint64_t)out_h * out_w;
    for (uint32_t ow = 0; ow < out_w; ++ow) {
        uint32_t valid_count = 0;                                   /* :122-131 */
        for (uint32_t khi = 0; khi < ph; ++khi)
            for (uint32_t kwi = 0; kwi < pw; ++kwi) {
                const int64_t ih = (int64_t)oh * sh + (int64_t)khi * dh - pad_top;
                const int64_t iw = (int64_t)ow * sw + (int64_t)kwi * dw - pad_left;
                if (ih >= 0 && ih < (int64_t)in_h && iw >= 0 && iw < (int64_t)in_w) valid_count++;
            }
        const uint32_t denom = cip ? ph * pw : valid_count;         /* :134-136 */
        for (uint32_t ct = 0; ct < c_tiles; ++ct) {
            const uint32_t c_off = ct * PL_TILE_C;
            const uint32_t c_valid = (ch - c_off) < PL_TILE_C ? (ch - c_off) : PL_TILE_C;
            for (uint32_t c1 = 0; c1 < c_valid; ++c1) {
                const int16_t *xc = x + ((uint64_t)ni * ch + c_off + c1) * hw;
                /* acc init :185-190: MAX -> kAccMin = -32768.0 (raw -2^31), else 0 */
                uint32_t acc = pool_type == 0 ? 0x80000000u : 0u;
                for (uint32_t khi = 0; khi < ph; ++khi) {
                    const int64_t ih = (int64_t)oh * sh + (int64_t)khi * dh - pad_top;
                    const int ih_ok = ih >= 0 && ih < (int64_t)in_h;
                    for (uint32_t kwi = 0; kwi < pw; ++kwi) {
                        const int64_t iw = (int64_t)ow * sw + (int64_t)kwi * dw - pad_left;
                        const int valid = ih_ok && iw >= 0 && iw < (int64_t)in_w;
                        /* pad fill :168-172: MAX -> kDataMin = -128.0 (raw -32768), else 0 */
                        const int16_t xv = valid ? xc[(uint64_t)ih * in_w + (uint64_t)iw]
                                                 : (int16_t)(pool_type == 0 ? -32768 : 0);
                        const uint32_t val = data_to_acc(xv);
                        if (pool_type == 0) {                       /* :214-215 */
                            if ((int32_t)val > (int32_t)acc) acc = val;
                        } else if (pool_type == 1) {                /* :216-217 */
                            acc += val;
                        } else if (lp_order == 1u) {                /* :222-223 */
                            acc += (int32_t)val < 0 ? (uint32_t)(-(int64_t)(int32_t)val) : val;
                        } else {                                    /* :224: AccData_t(val*val) = x^2 raw */
                            acc += (uint32_t)((int32_t)xv * (int32_t)xv);
                        }
                    }
                }
                int16_t out;                                        /* :253-266 */
                if (pool_type == 0) out = acc_to_data(acc);
                else if (pool_type == 1) out = ora_avg_finalize(acc, denom);
                else out = (lp_order == 1u) ? acc_to_data(acc) : ora_lp2_finalize(acc);
                y[((uint64_t)ni * ch + c_off + c1) * ohw + (uint64_t)oh * out_w + ow] = out;
            }
        }
    }
}

void ora_pool(const int16_t *x, int16_t *y, uint32_t batch, uint32_t ch,
              uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
              uint32_t ph, uint32_t pw, uint32_t sh, uint32_t sw,
              uint32_t pad_top, uint32_t pad_left, uint32_t dh, uint32_t dw,
              uint32_t pool_type, uint32_t lp_order, uint32_t cip) {
    for (uint32_t ni = 0; ni < batch; ++ni)                         /* :112 */
        for (uint32_t oh = 0; oh < out_h; ++oh)
            pool_row(x, y, ni, oh, ch, in_h, in_w, out_h, out_w, ph, pw, sh, sw,
                     pad_top, pad_left, dh, dw, pool_type, lp_order, cip);
}

void ora_pool_omp(const int16_t *x, int16_t *y, uint32_t batch, uint32_t ch,
                  uint32_t in_h, uint32_t in_w, uint32_t out_h, uint32_t out_w,
                  uint32_t ph, uint32_t pw, uint32_t sh, uint32_t sw,
                  uint32_t pad_top, uint32_t pad_left, uint32_t dh, uint32_t dw,
                  uint32_t pool_type, uint32_t lp_order, uint32_t cip) {
    const int64_t units = (int64_t)batch * out_h;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t u = 0; u < units; ++u)
        pool_row(x, y, (uint32_t)(u / out_h), (uint32_t)(u % out_h), ch, in_h, in_w, out_h,
                 out_w, ph, pw, sh, sw, pad_top, pad_left, dh, dw, pool_type, lp_order, cip);
}

void ora_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int ora_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
