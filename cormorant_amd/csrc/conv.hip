// conv.hip -- ConvKernel for gfx950 (kernels/conv/kernel/ConvKernel.cpp:46-343).
//
// Dispatch (standard convolutions, first match):
//   * few output channels, K <= 32, many pixels: direct vector-ALU kernel;
//   * windows of >= 2 taps, the same stride and dilation on both axes, when the
//     caller's workspace holds the packed weights: conv_pgemm (input patch in
//     LDS, weights pre-split into limb planes; conv_pgemm.hip);
//   * 3x3, <= 64 channels in and out, stride 1 or 2: conv_patch (input patch and
//     all weights in LDS);
//   * 1x1 / stride 1 / no padding, planes that fill 128-column tiles: batched
//     GEMM Y[n] = W[out_ch][in_ch] x X[n][in_ch][h*w] on the int8-limb MFMA core;
//   * any other: implicit GEMM on the same core, im2col gathered straight from
//     NCHW x while the B tile is built (no im2col buffer);
//   * depthwise (is_depthwise = 1, weights [out_ch][1][kh][kw]): direct kernel,
//     one thread per output, uint32 wrapping accumulator (ConvKernel.cpp:251-319).
// All paths: acc = wrap32((has_bias ? bias << 8 : 0) + sum x*w), y = sat16(acc >> 8),
// then the optional fused epilogue (Add of a same-shaped tensor, Relu / Relu6).
#include "cm_internal.h"
#include "q88.h"

int cm_conv_gemm_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                        uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                        uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                        uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                        uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc);
int cm_conv_pointwise_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                             uint32_t batch, uint32_t in_ch, uint32_t out_ch, uint32_t hw,
                             const cm_epilogue_t* epi, const LaunchCtx& lc);
int cm_conv_pgemm_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                         uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                         uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                         uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                         uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc);

namespace {

constexpr int kThreads = 256;

struct DwGeom {
    uint32_t in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pt, pl;
};

// Depthwise: output channel m reads input channel m of the same image.
template <bool HAS_BIAS>
__global__ __launch_bounds__(kThreads) void conv_depthwise(const int16_t* __restrict__ x,
                                                           const int16_t* __restrict__ w,
                                                           const int16_t* __restrict__ bias,
                                                           int16_t* __restrict__ y, DwGeom g,
                                                           uint64_t total, EpiArgs epi) {
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
// a broadcast), next to a per-k table of input byte offsets and tap numbers.
constexpr int kDirThreads = 256;
constexpr uint32_t kDirChunk = 8;   // k values gathered per load batch

struct DirArgs {
    const int16_t* x;
    const int16_t* w;
    const int16_t* bias;
    int16_t* y;
    uint32_t M, H, W, P, OW, kh, kw, sh, sw, dh, dw, pt, pl;
    uint32_t K, Kc;          // C*kh*kw; K rounded up to 2*kDirChunk
    uint32_t npix;           // batch * P
    uint32_t x_bytes;        // whole input tensor, < 2^31
    uint32_t x_img;          // C*H*W
    uint64_t y_img;          // M*P
    FastDiv div_p, div_ow, div_kk, div_kw;
    EpiArgs epi;
};

typedef short v2s __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t dot2(uint32_t x, uint32_t w, uint32_t acc) {
    return (uint32_t)__builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, x), __builtin_bit_cast(v2s, w),
                                            (int)acc, false);
}

template <int MT, bool HAS_BIAS>
__global__ __launch_bounds__(kDirThreads) void conv_direct(DirArgs g) {
    extern __shared__ __align__(16) uint32_t dsm[];
    uint32_t* wt = dsm;                                          // [Kc / 2][MT]
    int2* tab = reinterpret_cast<int2*>(dsm + (g.Kc / 2) * MT);   // [Kc + kDirChunk]
    // bias << 8 of the block's channels, staged with the weights so that the
    // epilogue does not start with a memory round trip
    uint32_t* bsm = reinterpret_cast<uint32_t*>(tab + g.Kc + kDirChunk);   // [MT]
    const uint32_t m0 = blockIdx.y * MT;
    // Weight words (k pair, channel): at most 16 x MT (K <= 32), two per thread.
    // Their loads and the bias load are buffer loads issued before anything is
    // stored, so one memory round trip covers them and overlaps the k table
    // below; taps past K and channels past M read 0 (offsets with bit 31 set).
    constexpr int WPT = (16 * MT + kDirThreads - 1) / kDirThreads;
    const uint32_t nwords = (g.Kc / 2) * MT;
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
    const uint32_t kk = g.kh * g.kw, hw = g.H * g.W;
    // k >= K (padding up to Kc, and one chunk past it that the last prefetch
    // reads) is tap 31, which every thread treats as outside the image
    for (uint32_t k = threadIdx.x; k < g.Kc + kDirChunk; k += kDirThreads) {
        const uint32_t c = fdiv(k, g.div_kk), r = k - c * kk;
        const uint32_t khi = fdiv(r, g.div_kw), kwi = r - khi * g.kw;
        tab[k] = k < g.K ? int2{(int)(2u * (c * hw + khi * g.dh * g.W + kwi * g.dw)), (int)r}
                         : int2{0, 31};
    }
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
        const uint32_t i = u * kDirThreads + threadIdx.x;
        if (i < nwords) wt[i] = wlo[u] | whi[u] << 16;
    }
    if (threadIdx.x < (uint32_t)MT) bsm[threadIdx.x] = bias_v;

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
    __syncthreads();

    uint32_t acc[MT];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) acc[mm] = 0u;
    auto load_chunk = [&](uint32_t k0, uint32_t (&xv)[kDirChunk]) {
#pragma unroll
        for (uint32_t q = 0; q < kDirChunk; ++q) {
            const int2 t = tab[k0 + q];
            const uint32_t off = (((holes >> t.y) & 1u) << 31) | (uint32_t)(pbyte + t.x);
            xv[q] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
        }
    };
    auto compute_chunk = [&](uint32_t k0, const uint32_t (&xv)[kDirChunk]) {
#pragma unroll
        for (uint32_t q = 0; q < kDirChunk / 2; ++q) {
            const uint32_t xp = xv[2 * q] | xv[2 * q + 1] << 16;
            const uint32_t* wr = wt + (k0 / 2 + q) * MT;
#pragma unroll
            for (int mm = 0; mm < MT; mm += 4) {
                const v4u wv = *reinterpret_cast<const v4u*>(wr + mm);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[mm + e] = dot2(xp, wv[e], acc[mm + e]);
            }
        }
    };
    // two gather batches in flight: the next one loads while this one computes
    // (loads are unconditional; the batch past the end reads only padding)
    uint32_t xa[kDirChunk], xb[kDirChunk];
    load_chunk(0, xa);
    for (uint32_t k0 = 0; k0 < g.Kc; k0 += 2 * kDirChunk) {
        load_chunk(k0 + kDirChunk, xb);
        __builtin_amdgcn_sched_barrier(0);   // keep the loads ahead of the compute
        compute_chunk(k0, xa);
        load_chunk(k0 + 2 * kDirChunk, xa);
        __builtin_amdgcn_sched_barrier(0);
        compute_chunk(k0 + kDirChunk, xb);
    }

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

template <int MT>
int launch_direct(const DirArgs& g, hipStream_t s) {
    const dim3 grid((g.npix + kDirThreads - 1) / kDirThreads, (g.M + MT - 1) / MT);
    const size_t lds = (size_t)(g.Kc / 2) * MT * 4u + (size_t)(g.Kc + kDirChunk) * 8u + MT * 4u;
    if (g.bias) hipLaunchKernelGGL((conv_direct<MT, true>), grid, dim3(kDirThreads), lds, s, g);
    else hipLaunchKernelGGL((conv_direct<MT, false>), grid, dim3(kDirThreads), lds, s, g);
    return cm_check_launch("conv_direct");
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
        g.Kc = (uint32_t)((K + 2 * kDirChunk - 1) / (2 * kDirChunk) * (2 * kDirChunk));
        g.npix = (uint32_t)npix;
        g.x_bytes = (uint32_t)x_bytes;
        g.x_img = in_ch * in_h * in_w;
        g.y_img = (uint64_t)out_ch * out_h * out_w;
        g.div_p = make_fastdiv(g.P);
        g.div_ow = make_fastdiv(out_w);
        g.div_kk = make_fastdiv(kh * kw);
        g.div_kw = make_fastdiv(kw);
        g.epi = ea;
        switch (mt) {
            case 8: return launch_direct<8>(g, s);
            case 16: return launch_direct<16>(g, s);
            case 24: return launch_direct<24>(g, s);
            default: return launch_direct<32>(g, s);
        }
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
    // 1x1 / stride 1 / no padding as one GEMM per image, when an image's
    // pixels fill its 128-column tiles to at least 80 %; small planes (e.g.
    // 7x7, 14x14) go through the gather path, whose columns run across images
    const uint64_t hw = (uint64_t)in_h * in_w;
    const uint64_t tiles = (hw + 127) / 128;
    if (kh == 1 && kw == 1 && sh == 1 && sw == 1 && pad_top == 0 && pad_left == 0 &&
        out_h == in_h && out_w == in_w && hw <= 0x7FFFFFFFull && (tiles * 128 - hw) * 5 <= tiles * 128)
        return cm_conv_pointwise_launch(x, w, b, y, batch, in_ch, out_ch, (uint32_t)hw, epi, lc);
    return cm_conv_gemm_launch(x, w, b, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                               sh, sw, dh, dw, pad_top, pad_left, epi, lc);
}
