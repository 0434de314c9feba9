// conv.hip -- ConvKernel for gfx950 (kernels/conv/kernel/ConvKernel.cpp:46-343).
//
// Dispatch (standard convolutions, first match):
//   * few output channels, K <= 32, many pixels: direct vector-ALU kernel;
//   * strided windows of 2..32 taps, small layers (<= 2^19 outputs, K <= 2048): one
//     block of four waves per 32x32 output tile, the reduction split over the
//     waves, fragments loaded straight into registers (conv_rk.hip);
//   * windows of >= 2 taps, the same stride and dilation on both axes, when the
//     caller's workspace holds the packed weights: conv_pgemm (input patch in
//     LDS, weights pre-split into limb planes; conv_pgemm.hip);
//   * 3x3, <= 64 channels in and out, stride 1 or 2: conv_patch (input patch and
//     all weights in LDS);
//   * 1x1 / stride 1 / no padding, small layers (<= 2^21 outputs, in_ch <= 512):
//     one wave per 32x32 output tile, fragments loaded straight into registers,
//     no LDS (conv_pw.hip);
//   * 1x1 / stride 1 / no padding, planes that fill 128-column tiles: batched
//     GEMM Y[n] = W[out_ch][in_ch] x X[n][in_ch][h*w] on the int8-limb MFMA core;
//   * any other: implicit GEMM on the same core, im2col gathered straight from
//     NCHW x while the B tile is built (no im2col buffer);
//   * depthwise (is_depthwise = 1, weights [out_ch][1][kh][kw]): LDS band kernel
//     (rows too wide for it: one thread per output), uint32 wrapping accumulator
//     (ConvKernel.cpp:251-319).
// All paths: acc = wrap32((has_bias ? bias << 8 : 0) + sum x*w), y = sat16(acc >> 8),
// then the optional fused epilogue (Add of a same-shaped tensor, Relu / Relu6).
#include "cm_internal.h"
#include "q88.h"

#include <algorithm>

int cm_conv_gemm_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                        uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                        uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                        uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                        uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc);
int cm_conv_pointwise_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                             uint32_t batch, uint32_t in_ch, uint32_t out_ch, uint32_t hw,
                             const cm_epilogue_t* epi, const LaunchCtx& lc);
int cm_conv_pw_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                      uint32_t batch, uint32_t in_ch, uint32_t out_ch, uint32_t hw,
                      const cm_epilogue_t* epi, const LaunchCtx& lc);
bool cm_conv_rk_takes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                      uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t sh, uint32_t sw,
                      uint32_t dh, uint32_t dw, uint32_t pad_top, uint32_t pad_left);
int cm_conv_rk_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y, uint32_t batch,
                      uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h,
                      uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t sh, uint32_t sw, uint32_t dh,
                      uint32_t dw, uint32_t pad_top, uint32_t pad_left, const cm_epilogue_t* epi,
                      const LaunchCtx& lc);
int cm_conv_pgemm_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                         uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                         uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                         uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                         uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc);

namespace {

constexpr int kThreads = 256;

// ---------------------------------------------------------------- depthwise --
// Output channel m of image n reads input channel m of image n through its own
// kh x kw filter (ConvKernel.cpp:251-319).  Work item = (image, channel, band of
// `band_h` output rows); one block per item.  The block stages the band's
// input rows in LDS with their zero padding -- tile row i holds input row
// ih_lo + i, tile column j holds input column j - cofs, out-of-range
// positions hold 0 -- so every tap reads LDS without a bounds check (a zero
// tap adds nothing to the wrapping sum, exactly like the reference's skipped
// tap).  Global reads are range-checked buffer loads (16-byte vectors when
// input rows are whole vectors), issued in batches before any is written to
// LDS.  A thread then owns one output column and a segment of the band's rows;
// for a 3x3 filter with row stride 1 it slides a 3-row window down the
// column, reading one new tile row per output.  The filter is block-uniform:
// its taps are scalar loads.  Products of two int16 values accumulate in
// uint32, wrapping mod 2^32 like AccData_t.
constexpr uint32_t kDwLdsBytes = 48u << 10;   // tile budget per block
constexpr int kDwBatch = 2;                   // staging loads in flight per thread and pass

struct DwBand {
    const int16_t* x;
    const int16_t* w;
    const int16_t* bias;
    int16_t* y;
    EpiArgs epi;
    uint32_t C, M, H, W, OH, OW, kh, kw, sh, sw, dh, dw, pt, pl;
    uint32_t band_h, n_bands;
    uint32_t pp, n_groups;        // channels (planes) per item, channel groups per image
    uint32_t pitch, cofs, rows;   // one plane's tile: rows x pitch elements, input column 0 at
                                  // cofs; a block stacks pp of them
    uint32_t vec;                 // 16-byte staging (W % 8 == 0, cofs and pitch % 8 == 0, x aligned)
    uint32_t units, gdr, gdj;     // staging units per tile row (pitch / 8 or pitch); a thread's
                                  // next unit is gdr rows and gdj units on (kThreads = gdr * units + gdj)
    uint32_t segs;                // row segments per column when pp * OW < kThreads, else 0
    FastDiv div_bands, div_groups, div_ow, div_units, div_cols, div_rows;   // div_cols: pp * OW
};

// Stage the input rows [ih_lo, ih_lo + rows) of planes 0..np-1 (consecutive
// channels, plane j at element j * plane of the resource): stacked tile row
// j * rows + r, unit u covers tile columns [u * E, u * E + E) (E = 8 for
// 16-byte units, else 1).
template <int E>
__device__ __forceinline__ void dw_stage(const DwBand& g, int16_t* tile, const __amdgpu_buffer_rsrc_t rs,
                                         int32_t ih_lo, uint32_t rows, const FastDiv& div_rows,
                                         uint32_t np) {
    typedef short v8s __attribute__((ext_vector_type(8)));
    const uint32_t n = np * rows * g.units, plane = g.H * g.W;
    uint32_t rr = fdiv(threadIdx.x, g.div_units);   // stacked row j * rows + r
    uint32_t u = threadIdx.x - rr * g.units;
    for (uint32_t base = 0; base < n; base += kThreads * kDwBatch) {
        uint32_t off[kDwBatch], dst[kDwBatch];
#pragma unroll
        for (int k = 0; k < kDwBatch; ++k) {
            const uint32_t j = fdiv(rr, div_rows), r = rr - j * rows;   // plane, row within it
            const int32_t ih = ih_lo + (int32_t)r, iw = (int32_t)(u * E) - (int32_t)g.cofs;
            const bool in = j < np;
            const bool ok = in && (uint32_t)ih < g.H && (uint32_t)iw < g.W;
            off[k] = ok ? (j * plane + (uint32_t)ih * g.W + (uint32_t)iw) * 2u : kOob;
            dst[k] = in ? rr * g.units + u : 0xFFFFFFFFu;
            rr += g.gdr;
            u += g.gdj;
            if (u >= g.units) {
                u -= g.units;
                ++rr;
            }
        }
        if constexpr (E == 8) {
            v8s d[kDwBatch];
#pragma unroll
            for (int k = 0; k < kDwBatch; ++k)
                d[k] = __builtin_bit_cast(v8s, __builtin_amdgcn_raw_buffer_load_b128(rs, off[k], 0, 0));
#pragma unroll
            for (int k = 0; k < kDwBatch; ++k)
                if (dst[k] != 0xFFFFFFFFu) *reinterpret_cast<v8s*>(tile + dst[k] * 8) = d[k];
        } else {
            int16_t d[kDwBatch];
#pragma unroll
            for (int k = 0; k < kDwBatch; ++k) d[k] = (int16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off[k], 0, 0);
#pragma unroll
            for (int k = 0; k < kDwBatch; ++k)
                if (dst[k] != 0xFFFFFFFFu) tile[dst[k]] = d[k];
        }
    }
}

template <int K, bool HAS_BIAS>   // K > 0: a K x K filter with dilation 1
__global__ __launch_bounds__(kThreads) void conv_dw_band(DwBand g) {
    extern __shared__ __align__(16) int16_t tile[];
    // volatile: element reads, never paired into unaligned 4-byte reads
    typedef __attribute__((address_space(3))) const volatile int16_t lds_i16;
    const uint32_t item = blockIdx.x;
    const uint32_t ng = fdiv(item, g.div_bands);        // n * n_groups + channel group
    const uint32_t band = item - ng * g.n_bands;
    const uint32_t n = fdiv(ng, g.div_groups);
    const uint32_t m0 = (ng - n * g.n_groups) * g.pp;
    const uint32_t np = min(g.pp, g.M - m0);
    const uint32_t oh0 = band * g.band_h;
    const uint32_t bh = min(g.band_h, g.OH - oh0);
    const int32_t ih_lo = (int32_t)(oh0 * g.sh) - (int32_t)g.pt;
    const uint32_t plane = g.H * g.W;
    const int16_t* xc = g.x + ((uint64_t)n * g.C + m0) * plane;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(xc, np * plane * 2u);
    // A thread owns one column of one plane and a segment of the band's rows
    // (or, when the block has >= kThreads columns, every kThreads-th column
    // over all rows).  Column q of the block is column q % OW of plane q / OW.
    const uint32_t ncols = g.pp * g.OW;
    uint32_t q0 = threadIdx.x, qstep = kThreads, ra = 0, rb = bh;
    if (g.segs > 0) {
        const uint32_t sgi = fdiv(threadIdx.x, g.div_cols);
        q0 = threadIdx.x - sgi * ncols;
        qstep = ncols;   // one column
        const uint32_t rps = (bh + g.segs - 1) / g.segs;
        ra = min(bh, sgi * rps);
        rb = sgi < g.segs ? min(bh, ra + rps) : ra;
    }
    // the first column's filter and bias load while the tile stages
    int32_t wk[K > 0 ? K * K : 1];
    uint32_t acc0 = 0, jl = 0xFFFFFFFFu;
    auto load_filter = [&](uint32_t j) {
        if constexpr (K > 0) {
            const int16_t* wm = g.w + (uint64_t)(m0 + j) * (K * K);
#pragma unroll
            for (int t = 0; t < K * K; ++t) wk[t] = wm[t];
        }
        acc0 = HAS_BIAS ? q88::data_to_acc(g.bias[m0 + j]) : 0u;
        jl = j;
    };
    if (g.pp == 1) {
        load_filter(0u);   // block-uniform: scalar loads
    } else if (q0 < ncols) {
        const uint32_t j = fdiv(q0, g.div_ow);
        if (j < np) load_filter(j);
    }
    // every band stages g.rows rows per plane (the last band's extra rows are
    // never read), so the stacked layout is the same for all items
    if (g.vec) dw_stage<8>(g, tile, rs, ih_lo, g.rows, g.div_rows, np);
    else dw_stage<1>(g, tile, rs, ih_lo, g.rows, g.div_rows, np);
    __syncthreads();
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    const uint32_t pitch = g.pitch, rstep = g.sh * pitch;
    for (uint32_t q = q0; q < ncols; q += qstep) {
        const uint32_t j = fdiv(q, g.div_ow), c = q - j * g.OW;
        if (j >= np) break;   // q only grows
        if (j != jl) load_filter(j);
        const uint32_t m = m0 + j;
        const int16_t* wm = g.w + (uint64_t)m * g.kh * g.kw;
        const uint64_t ybase = (((uint64_t)n * g.M + m) * g.OH + oh0) * g.OW;
        int16_t* yb = g.y + ybase;
        const int16_t* addb = g.epi.add_mode == 1u ? g.epi.add + ybase : nullptr;
        const int16_t* tp = tile + j * g.rows * pitch + c * g.sw + (g.cofs - g.pl);
        if constexpr (K > 0) {
            if (g.sh == 1) {
                // sliding window down the column: each output row reads one new tile row
                int32_t v[K][K];
                lds_i16* t = (lds_i16*)(tp + ra * pitch);
#pragma unroll
                for (int khi = 0; khi < K - 1; ++khi)
#pragma unroll
                    for (int kwi = 0; kwi < K; ++kwi) v[khi + 1][kwi] = t[khi * pitch + kwi];
                t += (K - 1) * pitch;
                for (uint32_t r = ra; r < rb; ++r) {
#pragma unroll
                    for (int khi = 0; khi < K - 1; ++khi)
#pragma unroll
                        for (int kwi = 0; kwi < K; ++kwi) v[khi][kwi] = v[khi + 1][kwi];
#pragma unroll
                    for (int kwi = 0; kwi < K; ++kwi) v[K - 1][kwi] = t[kwi];
                    t += pitch;
                    uint32_t acc = acc0;
#pragma unroll
                    for (int khi = 0; khi < K; ++khi)
#pragma unroll
                        for (int kwi = 0; kwi < K; ++kwi) acc += (uint32_t)(v[khi][kwi] * wk[khi * K + kwi]);
                    int32_t o = q88::acc_to_data(acc);
                    if (addb) o = q88::add(o, addb[r * g.OW + c]);
                    yb[r * g.OW + c] = (int16_t)q88::clamp(o, lo, hi);
                }
                continue;
            }
        }
        for (uint32_t r = ra; r < rb; ++r) {
            lds_i16* t = (lds_i16*)(tp + r * rstep);
            uint32_t acc = acc0;
            if constexpr (K > 0) {
#pragma unroll
                for (int khi = 0; khi < K; ++khi)
#pragma unroll
                    for (int kwi = 0; kwi < K; ++kwi)
                        acc += (uint32_t)((int32_t)t[khi * pitch + kwi] * wk[khi * K + kwi]);
            } else {
                for (uint32_t khi = 0; khi < g.kh; ++khi) {
                    lds_i16* tr = t + khi * g.dh * pitch;
                    const int16_t* wr = wm + khi * g.kw;
                    for (uint32_t kwi = 0; kwi < g.kw; ++kwi)
                        acc += (uint32_t)((int32_t)tr[kwi * g.dw] * (int32_t)wr[kwi]);
                }
            }
            int32_t o = q88::acc_to_data(acc);
            if (addb) o = q88::add(o, addb[r * g.OW + c]);
            yb[r * g.OW + c] = (int16_t)q88::clamp(o, lo, hi);
        }
    }
}

// Band geometry of a depthwise convolution; false when one output row's input
// rows do not fit the LDS budget or indices leave 32-bit range (the per-output
// kernel below takes those shapes).
bool dw_band_geom(DwBand& g, uint64_t batch, uintptr_t xaddr) {
    const uint64_t iw_max = (uint64_t)(g.OW - 1) * g.sw + (uint64_t)(g.kw - 1) * g.dw;   // + pl offset
    const uint64_t planes = batch * g.M;
    if ((uint64_t)g.H * g.W >= (1u << 26) || g.OW >= (1u << 24) || g.OH >= (1u << 24) || g.pl >= (1u << 20) ||
        iw_max >= (1u << 24) || planes >= (1u << 30) ||
        (uint64_t)g.OH * g.sh + g.pt + (uint64_t)g.kh * g.dh >= (1u << 30))
        return false;
    g.cofs = (g.pl + 7) & ~7u;
    const uint64_t need_cols = std::max<uint64_t>(g.W, iw_max + 1 > g.pl ? iw_max + 1 - g.pl : 0);
    const uint64_t pitch = (g.cofs + need_cols + 7) & ~7ull;
    auto rows_of = [&](uint64_t bh) { return (bh - 1) * g.sh + (uint64_t)(g.kh - 1) * g.dh + 1; };
    if (rows_of(1) * pitch * 2 > kDwLdsBytes) return false;
    g.pitch = (uint32_t)pitch;
    // About four outputs per thread, as long as the grid keeps four blocks per
    // CU: bands of one plane's rows, or, when a whole plane is fewer outputs
    // than that, several consecutive channels' planes per block.
    const uint64_t want = 4ull * cm_cu_count(), per_block = 4ull * kThreads;
    uint64_t bh = std::min<uint64_t>(g.OH, (per_block + g.OW - 1) / g.OW);
    while (bh > 1 && planes * ((g.OH + bh - 1) / bh) < want) bh = (bh + 1) / 2;
    while (bh > 1 && rows_of(bh) * pitch * 2 > kDwLdsBytes) --bh;
    g.band_h = (uint32_t)std::max<uint64_t>(bh, 1);
    g.n_bands = (g.OH + g.band_h - 1) / g.band_h;
    g.rows = (uint32_t)rows_of(g.band_h);
    uint64_t pp = 1;
    if (g.n_bands == 1) {
        const uint64_t outs = (uint64_t)g.OH * g.OW, tile_bytes = (uint64_t)g.rows * pitch * 2;
        pp = std::max<uint64_t>(1, std::min<uint64_t>({per_block / outs, (uint64_t)g.M, kDwLdsBytes / tile_bytes}));
        while (pp > 1 && batch * ((g.M + pp - 1) / pp) < want) pp = (pp + 1) / 2;
    }
    g.pp = (uint32_t)pp;
    g.n_groups = (uint32_t)((g.M + pp - 1) / pp);
    if (batch * g.n_groups * g.n_bands > 0x7FFFFFFFull || pp * g.H * g.W >= (1u << 30)) return false;
    g.vec = g.W % 8 == 0 && (xaddr & 15u) == 0;
    g.units = g.vec ? g.pitch / 8 : g.pitch;
    g.gdr = kThreads / g.units;
    g.gdj = kThreads % g.units;
    const uint64_t ncols = pp * g.OW;
    g.segs = ncols < kThreads ? (uint32_t)(kThreads / ncols) : 0u;
    g.div_bands = make_fastdiv(g.n_bands);
    g.div_groups = make_fastdiv(g.n_groups);
    g.div_ow = make_fastdiv(g.OW);
    g.div_units = make_fastdiv(g.units);
    g.div_rows = make_fastdiv(g.rows);
    g.div_cols = make_fastdiv((uint32_t)std::min<uint64_t>(ncols, 0x7FFFFFFF));
    return true;
}

struct DwGeom {
    uint32_t in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pt, pl;
};

// Per-output fallback for rows too wide for the band tile: one thread per output.
template <bool HAS_BIAS>
__global__ __launch_bounds__(kThreads) void conv_depthwise(const int16_t* __restrict__ x,
                                                           const int16_t* __restrict__ w,
                                                           const int16_t* __restrict__ bias,
                                                           int16_t* __restrict__ y, DwGeom g,
                                                           uint64_t total, EpiArgs epi) {
    touch_lines(g, epi);
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    const uint64_t ohw = (uint64_t)g.out_h * g.out_w;
    for (uint64_t o = (uint64_t)blockIdx.x * kThreads + threadIdx.x; o < total; o += stride) {
        const uint64_t nm = o / ohw;                       // n * out_ch + m
        const uint32_t rem = (uint32_t)(o - nm * ohw);
        const uint64_t n = nm / g.out_ch;
        const uint32_t m = (uint32_t)(nm - n * g.out_ch);
        const uint32_t oh = rem / g.out_w, ow = rem - (rem / g.out_w) * g.out_w;
        const int16_t* xc = x + (n * g.in_ch + m) * (uint64_t)g.in_h * g.in_w;
        const int16_t* wm = w + (uint64_t)m * g.kh * g.kw;
        uint32_t acc = HAS_BIAS ? q88::data_to_acc(bias[m]) : 0u;
        const int64_t ih0 = (int64_t)oh * g.sh - g.pt, iw0 = (int64_t)ow * g.sw - g.pl;
        for (uint32_t khi = 0; khi < g.kh; ++khi) {
            const int64_t ih = ih0 + (int64_t)khi * g.dh;
            if (ih < 0 || ih >= (int64_t)g.in_h) continue;
            for (uint32_t kwi = 0; kwi < g.kw; ++kwi) {
                const int64_t iw = iw0 + (int64_t)kwi * g.dw;
                if (iw < 0 || iw >= (int64_t)g.in_w) continue;
                acc += (uint32_t)((int32_t)xc[(uint64_t)ih * g.in_w + iw] * (int32_t)wm[khi * g.kw + kwi]);
            }
        }
        int32_t v = q88::acc_to_data(acc);
        if (epi.add_mode == 1u) v = q88::add(v, epi.add[o]);
        y[o] = (int16_t)q88::epi_act(v, epi.act);
    }
}

// ------------------------------------------------------------------ direct --
// Standard convolution with few output channels on the vector ALUs.  The
// int8-limb MFMA path works on 128 output channels x 128 pixels per block;
// with 16-32 output channels most of that tile is empty, and each block's
// fixed costs (operand staging, LDS round trips, the epilogue) dominate.  Here
// a thread owns one output pixel (flattened over the images) and MT output
// channels: it walks k = (c, kh, kw) two at a time, gathers the two input values
// (one buffer load each, padding taps are sent out of the buffer range and read
// 0), and accumulates w*x for all MT channels with v_dot2 (int16 x int16 pairs
// into the int32 accumulator, wrapping mod 2^32 like the reference's).
// Weights of the block's MT channels sit in LDS as [k pair][MT] words (read as
// a broadcast).  With K <= 32 every gather of a thread and the block's weight
// loads are issued together at the start: the offsets of the k values depend on
// the shape alone (a table in the kernel arguments), so one memory round trip
// covers them all.
constexpr int kDirThreads = 256;
constexpr uint32_t kDirChunk = 16;   // K is rounded up to a multiple of this (KC = 16 or 32)

struct DirArgs {
    const int16_t* x;
    const int16_t* w;
    const int16_t* bias;
    int16_t* y;
    uint32_t M, H, W, P, OW, kh, kw, sh, sw, dh, dw, pt, pl;
    uint32_t K, Kc;          // C*kh*kw; K rounded up to kDirChunk
    uint32_t npix;           // batch * P
    uint32_t x_bytes;        // whole input tensor, < 2^31
    uint32_t x_img;          // C*H*W
    uint64_t y_img;          // M*P
    FastDiv div_p, div_ow, div_kk, div_kw;
    EpiArgs epi;
    int32_t toff[32];        // per k = (c, tap): byte offset from the window origin
    uint8_t tap[32];         // per k: its tap, 31 past K (always padding)
};

typedef short v2s __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t dot2(uint32_t x, uint32_t w, uint32_t acc) {
    return (uint32_t)__builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, x), __builtin_bit_cast(v2s, w),
                                            (int)acc, false);
}

template <int MT, int KC, bool HAS_BIAS>
__global__ __launch_bounds__(kDirThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void conv_direct(DirArgs g) {
    touch_lines(g);
    extern __shared__ __align__(16) uint32_t dsm[];
    uint32_t* wt = dsm;                                                  // [KC / 2][MT]
    // bias << 8 of the block's channels, staged with the weights so that the
    // epilogue does not start with a memory round trip
    uint32_t* bsm = dsm + (KC / 2) * MT;                                 // [MT]
    const uint32_t m0 = blockIdx.y * MT;
    // Weight words (k pair, channel): KC / 2 x MT, WPT per thread.  Buffer loads
    // with taps past K and channels past M sent out of range (bit 31), read 0.
    constexpr int WPT = ((KC / 2) * MT + kDirThreads - 1) / kDirThreads;
    constexpr uint32_t nwords = (KC / 2) * MT;
    uint32_t wlo[WPT], whi[WPT];
    {
        const __amdgpu_buffer_rsrc_t wr = make_rsrc(g.w, g.M * g.K * 2u);
#pragma unroll
        for (int u = 0; u < WPT; ++u) {
            const uint32_t i = u * kDirThreads + threadIdx.x;
            const uint32_t kp = i / MT, mm = i - kp * MT;
            const uint32_t m = m0 + mm, k = 2 * kp;
            const uint32_t ok = (uint32_t)(i < nwords) & (uint32_t)(m < g.M);
            const uint32_t base = ((m * g.K + k) * 2u) & 0x7FFFFFFFu;
            const uint32_t ok_lo = ok & (uint32_t)(k < g.K), ok_hi = ok & (uint32_t)(k + 1 < g.K);
            wlo[u] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(wr, base | ((ok_lo ^ 1u) << 31), 0, 0);
            whi[u] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(wr, (base + 2u) | ((ok_hi ^ 1u) << 31), 0, 0);
        }
    }
    uint32_t bias_v = 0;
    if constexpr (HAS_BIAS) {
        const __amdgpu_buffer_rsrc_t br = make_rsrc(g.bias, g.M * 2u);
        const uint32_t m = min(m0 + threadIdx.x, g.M - 1u);
        bias_v = q88::data_to_acc((int32_t)(int16_t)__builtin_amdgcn_raw_buffer_load_b16(br, m * 2u, 0, 0));
    }

    const uint32_t kk = g.kh * g.kw;
    const uint32_t pix = blockIdx.x * kDirThreads + threadIdx.x;
    const bool pok = pix < g.npix;
    const uint32_t n = pok ? fdiv(pix, g.div_p) : 0u;
    const uint32_t p = pok ? pix - n * g.P : 0u;
    const uint32_t oh = fdiv(p, g.div_ow), ow = p - oh * g.OW;
    const int32_t ih0 = (int32_t)(oh * g.sh) - (int32_t)g.pt;
    const int32_t iw0 = (int32_t)(ow * g.sw) - (int32_t)g.pl;
    uint32_t holes = 0x80000000u;   // bit r: tap r of this pixel's window is padding
    for (uint32_t r = 0; r < kk; ++r) {
        const uint32_t khi = fdiv(r, g.div_kw), kwi = r - khi * g.kw;
        const int32_t ih = ih0 + (int32_t)(khi * g.dh), iw = iw0 + (int32_t)(kwi * g.dw);
        const bool in = pok && ih >= 0 && ih < (int32_t)g.H && iw >= 0 && iw < (int32_t)g.W;
        holes |= in ? 0u : 1u << r;
    }
    // byte offset of the window origin (negative when it starts in the padding;
    // only taps inside the image are ever added to it unmasked)
    const int32_t pbyte = 2 * ((int32_t)(n * g.x_img) + ih0 * (int32_t)g.W + iw0);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int16_t*>(g.x), (short)0, (int)g.x_bytes, 0x00020000);
    // every k value of the window: k = (c, tap), tap r = (kh, kw); k >= K is
    // tap 31, which every pixel treats as padding
    uint32_t xv[KC];
#pragma unroll
    for (uint32_t k = 0; k < (uint32_t)KC; ++k) {
        const uint32_t tap = g.tap[k];
        const uint32_t off = (((holes >> tap) & 1u) << 31) | ((uint32_t)(pbyte + g.toff[k]) & 0x7FFFFFFFu);
        xv[k] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
        const uint32_t i = u * kDirThreads + threadIdx.x;
        if (i < nwords) wt[i] = wlo[u] | whi[u] << 16;
    }
    if (threadIdx.x < (uint32_t)MT) bsm[threadIdx.x] = bias_v;
    __syncthreads();

    uint32_t acc[MT];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[mm] = 0u;
    // per k pair: all MT weight words read first (MT / 4 broadcast LDS reads in
    // flight together), then the MT dot products -- one LDS round trip per pair
#pragma unroll
    for (uint32_t q = 0; q < (uint32_t)KC / 2; ++q) {
        const uint32_t xp = xv[2 * q] | xv[2 * q + 1] << 16;
        const uint32_t* wr = wt + q * MT;
        v4u wv[MT / 4];
#pragma unroll
        for (int g4 = 0; g4 < MT / 4; ++g4) wv[g4] = *reinterpret_cast<const v4u*>(wr + 4 * g4);
#pragma unroll
        for (int g4 = 0; g4 < MT / 4; ++g4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[4 * g4 + e] = dot2(xp, wv[g4][e], acc[4 * g4 + e]);
        }
    }
    // the products are done here: without the empty asm the compiler sinks them
    // into the per-channel stores behind the pixel test below, keeping every
    // weight read live until then (KC * MT * 2 registers)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) asm volatile("" : "+v"(acc[mm]));

    if (!pok) return;
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    const uint64_t ybase = (uint64_t)n * g.y_img + p;
    // the fused Add's values for all MT channels first (channels past M read the
    // last one), so the loads are in flight together rather than one per store
    int32_t res[MT];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) res[mm] = 0;
    if (g.epi.add_mode == 1u) {
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) {
            const uint32_t m = min(m0 + mm, g.M - 1u);
            res[mm] = g.epi.add[ybase + (uint64_t)m * g.P];
        }
    }
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
        const uint32_t m = m0 + mm;
        uint32_t v = acc[mm];
        if (HAS_BIAS) v += bsm[mm];
        const int32_t yv = q88::clamp(q88::add(q88::acc_to_data(v), res[mm]), lo, hi);
        if (m < g.M) g.y[ybase + (uint64_t)m * g.P] = (int16_t)yv;
    }
}

// Output channels per thread for the direct path, or 0 when the MFMA path
// suits the shape better.  The direct path pays per multiply-add (v_dot2 plus
// a broadcast LDS read of the weights), the MFMA path per 128 x 128 tile; the
// direct one wins for few output channels with a short k range (e.g. a 3-channel
// stem, 1x1 convolutions of 16-32 channels) over enough pixels to fill the GPU.
uint32_t direct_channels(uint64_t K, uint32_t out_ch, uint32_t kk, uint64_t npix, uint64_t x_bytes) {
    if (out_ch > 32 || K > 32 || npix < 32768 || kk > 31 || x_bytes >= 0x80000000ull) return 0;
    return out_ch <= 8 ? 8 : out_ch <= 16 ? 16 : out_ch <= 24 ? 24 : 32;
}

template <int MT, int KC>
int launch_direct_kc(const DirArgs& g, hipStream_t s) {
    const dim3 grid((g.npix + kDirThreads - 1) / kDirThreads, (g.M + MT - 1) / MT);
    const size_t lds = (size_t)(KC / 2) * MT * 4u + MT * 4u;
    if (g.bias) hipLaunchKernelGGL((conv_direct<MT, KC, true>), grid, dim3(kDirThreads), lds, s, g);
    else hipLaunchKernelGGL((conv_direct<MT, KC, false>), grid, dim3(kDirThreads), lds, s, g);
    return cm_check_launch("conv_direct");
}

template <int MT>
int launch_direct(const DirArgs& g, hipStream_t s) {
    return g.Kc <= 16u ? launch_direct_kc<MT, 16>(g, s) : launch_direct_kc<MT, 32>(g, s);
}

}  // namespace

// The patch GEMM's 16-byte row staging: rows of whole 16-byte groups, x
// aligned, and gcd(stride, dilation) 1 or 2.
bool pgemm_row_loads(const int16_t* x, uint32_t in_w, uint32_t sh, uint32_t dh) {
    uint32_t a = sh, c = dh;
    while (c) { const uint32_t t = a % c; a = c; c = t; }
    return in_w % 8 == 0 && ((uintptr_t)x & 15) == 0 && (a == 1 || a == 2);
}

size_t cm_conv_packed_bytes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                            uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                            uint32_t kw, uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
                            uint32_t pad_top, uint32_t pad_left, uint32_t is_dw) {
    // the dispatch below: the patch-GEMM path comes after the direct one and
    // takes windows of two or more taps
    if (is_dw || kh * kw < 2) return 0;
    const uint64_t K = (uint64_t)in_ch * kh * kw;
    if (direct_channels(K, out_ch, kh * kw, (uint64_t)batch * out_h * out_w,
                        2ull * in_ch * in_h * in_w * batch))
        return 0;
    if (cm_conv_rk_takes(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top,
                         pad_left))
        return 0;
    alignas(16) static const int16_t probe[8] = {};   // an aligned stand-in, never read
    if (!pgemm_row_loads(probe, in_w, sh, dh)) {
        size_t need = 0;
        const LaunchCtx lc{nullptr, nullptr, 0, &need};
        if (cm_conv_patch_launch(probe, probe, probe, const_cast<int16_t*>(probe), batch, in_ch, in_h,
                                 in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left,
                                 nullptr, lc) == CM_OK)
            return 0;
    }
    return cm_conv_pgemm_packed_bytes(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw,
                                      dh, dw, pad_top, pad_left);
}

int cm_conv_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                   uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                   uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                   uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                   uint32_t pad_left, uint32_t has_bias, uint32_t is_dw, const cm_epilogue_t* epi,
                   const LaunchCtx& lc) {
    const hipStream_t s = lc.s;
    const int16_t* b = has_bias ? bias : nullptr;
    const EpiArgs ea = cm_epi_args(epi);
    if (is_dw) {
        const uint64_t total = (uint64_t)batch * out_ch * out_h * out_w;
        if (total == 0 || lc.need) return CM_OK;
        DwBand bg{};
        bg.x = x; bg.w = w; bg.bias = b; bg.y = y; bg.epi = ea;
        bg.C = in_ch; bg.M = out_ch; bg.H = in_h; bg.W = in_w; bg.OH = out_h; bg.OW = out_w;
        bg.kh = kh; bg.kw = kw; bg.sh = sh; bg.sw = sw; bg.dh = dh; bg.dw = dw; bg.pt = pad_top; bg.pl = pad_left;
        if (dw_band_geom(bg, batch, (uintptr_t)x)) {
            const dim3 grid((uint32_t)((uint64_t)batch * bg.n_groups * bg.n_bands));
            const size_t lds = (size_t)bg.pp * bg.rows * bg.pitch * 2;
            const bool k3 = kh == 3 && kw == 3 && dh == 1 && dw == 1;
            if (k3 && b) hipLaunchKernelGGL((conv_dw_band<3, true>), grid, dim3(kThreads), lds, s, bg);
            else if (k3) hipLaunchKernelGGL((conv_dw_band<3, false>), grid, dim3(kThreads), lds, s, bg);
            else if (b) hipLaunchKernelGGL((conv_dw_band<0, true>), grid, dim3(kThreads), lds, s, bg);
            else hipLaunchKernelGGL((conv_dw_band<0, false>), grid, dim3(kThreads), lds, s, bg);
            return cm_check_launch("conv_dw_band");
        }
        DwGeom g{in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left};
        const dim3 grid((uint32_t)cm_grid_blocks(total, kThreads));
        if (b) hipLaunchKernelGGL(conv_depthwise<true>, grid, dim3(kThreads), 0, s, x, w, b, y, g, total, ea);
        else hipLaunchKernelGGL(conv_depthwise<false>, grid, dim3(kThreads), 0, s, x, w, b, y, g, total, ea);
        return cm_check_launch("conv_depthwise");
    }
    const uint64_t K = (uint64_t)in_ch * kh * kw;
    const uint64_t x_bytes = 2ull * in_ch * in_h * in_w * batch;
    const uint64_t npix = (uint64_t)batch * out_h * out_w;
    if (const uint32_t mt = direct_channels(K, out_ch, kh * kw, npix, x_bytes)) {
        if (npix == 0 || out_ch == 0 || lc.need) return CM_OK;
        if (npix > 0x7FFFFFFFull) return cm_set_error(CM_ERR_RANGE, "conv: shape exceeds 32-bit indexing");
        DirArgs g{};
        g.x = x; g.w = w; g.bias = b; g.y = y;
        g.M = out_ch; g.H = in_h; g.W = in_w; g.P = out_h * out_w; g.OW = out_w;
        g.kh = kh; g.kw = kw; g.sh = sh; g.sw = sw; g.dh = dh; g.dw = dw; g.pt = pad_top; g.pl = pad_left;
        g.K = (uint32_t)K;
        g.Kc = (uint32_t)((K + kDirChunk - 1) / kDirChunk * kDirChunk);
        g.npix = (uint32_t)npix;
        g.x_bytes = (uint32_t)x_bytes;
        g.x_img = in_ch * in_h * in_w;
        g.y_img = (uint64_t)out_ch * out_h * out_w;
        g.div_p = make_fastdiv(g.P);
        g.div_ow = make_fastdiv(out_w);
        g.div_kk = make_fastdiv(kh * kw);
        g.div_kw = make_fastdiv(kw);
        g.epi = ea;
        for (uint32_t k = 0; k < 32; ++k) {
            const uint32_t c = k / (kh * kw), r = k % (kh * kw), khi = r / kw, kwi = r % kw;
            g.toff[k] = k < K ? (int32_t)(2u * (c * in_h * in_w + khi * dh * in_w + kwi * dw)) : 0;
            g.tap[k] = (uint8_t)(k < K ? r : 31u);
        }
        switch (mt) {
            case 8: return launch_direct<8>(g, s);
            case 16: return launch_direct<16>(g, s);
            case 24: return launch_direct<24>(g, s);
            default: return launch_direct<32>(g, s);
        }
    }
    // Small layers: the register-only kernel with the reduction split over a
    // block's waves (conv_rk.hip)
    if (cm_conv_rk_takes(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top,
                         pad_left)) {
        const int rc = cm_conv_rk_launch(x, w, b, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                                         sh, sw, dh, dw, pad_top, pad_left, epi, lc);
        if (rc != 1) return rc;
    }
    // The patch GEMM (it needs the caller's workspace for the packed weights)
    // stages input rows 16 bytes at a time when they allow it; where they do
    // not, conv_patch comes first when it takes the shape
    bool patch_tried = false;
    auto try_patch = [&]() {
        patch_tried = true;
        return cm_conv_patch_launch(x, w, b, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                                    sh, sw, dh, dw, pad_top, pad_left, epi, lc);
    };
    if (kh * kw > 1) {
        if (!pgemm_row_loads(x, in_w, sh, dh)) {
            const int rc = try_patch();
            if (rc != 1) return rc;
        }
        const int rc = cm_conv_pgemm_launch(x, w, b, y, batch, in_ch, in_h, in_w, out_ch, out_h,
                                            out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left, epi, lc);
        if (rc != 1) return rc;
    }
    if (!patch_tried) {   // 3x3 with <= 64 channels in and out: all weights staged per block
        const int rc = try_patch();
        if (rc != 1) return rc;
    }
    // 1x1 / stride 1 / no padding: small layers on the register-only MFMA kernel
    // (conv_pw.hip); else one GEMM per image, when an image's pixels fill its
    // 128-column tiles to at least 80 %; small planes (e.g. 7x7, 14x14) go
    // through the gather path, whose columns run across images
    const uint64_t hw = (uint64_t)in_h * in_w;
    const uint64_t tiles = (hw + 127) / 128;
    const bool pointwise = kh == 1 && kw == 1 && sh == 1 && sw == 1 && pad_top == 0 && pad_left == 0 &&
                           out_h == in_h && out_w == in_w && hw <= 0x7FFFFFFFull;
    if (pointwise) {
        const int rc = cm_conv_pw_launch(x, w, b, y, batch, in_ch, out_ch, (uint32_t)hw, epi, lc);
        if (rc != 1) return rc;
    }
    if (pointwise && (tiles * 128 - hw) * 5 <= tiles * 128)
        return cm_conv_pointwise_launch(x, w, b, y, batch, in_ch, out_ch, (uint32_t)hw, epi, lc);
    return cm_conv_gemm_launch(x, w, b, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                               sh, sw, dh, dw, pad_top, pad_left, epi, lc);
}
