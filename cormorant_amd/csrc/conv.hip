// conv.hip -- ConvKernel for gfx950 (kernels/conv/kernel/ConvKernel.cpp:46-343).
//
// Dispatch:
//   * standard conv, 1x1 / stride 1 / no padding, planes that fill 128-column
//     tiles: batched GEMM Y[n] = W[out_ch][in_ch] x X[n][in_ch][h*w] on the
//     int8-limb MFMA core;
//   * any other standard conv: implicit GEMM on the same core, im2col gathered
//     straight from NCHW x while the B tile is built (no im2col buffer);
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
                        uint32_t pad_left, const cm_epilogue_t* epi, hipStream_t s);
int cm_conv_pointwise_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                             uint32_t batch, uint32_t in_ch, uint32_t out_ch, uint32_t hw,
                             const cm_epilogue_t* epi, hipStream_t s);

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

}  // namespace

int cm_conv_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                   uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                   uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                   uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                   uint32_t pad_left, uint32_t has_bias, uint32_t is_dw, const cm_epilogue_t* epi,
                   hipStream_t s) {
    const int16_t* b = has_bias ? bias : nullptr;
    const EpiArgs ea = cm_epi_args(epi);
    if (is_dw) {
        const uint64_t total = (uint64_t)batch * out_ch * out_h * out_w;
        if (total == 0) return CM_OK;
        DwGeom g{in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left};
        const dim3 grid((uint32_t)cm_grid_blocks(total, kThreads));
        if (b) hipLaunchKernelGGL(conv_depthwise<true>, grid, dim3(kThreads), 0, s, x, w, b, y, g, total, ea);
        else hipLaunchKernelGGL(conv_depthwise<false>, grid, dim3(kThreads), 0, s, x, w, b, y, g, total, ea);
        return cm_check_launch("conv_depthwise");
    }
    // 1x1 / stride 1 / no padding as one GEMM per image, when an image's
    // pixels fill its 128-column tiles to at least 80 %; small planes (e.g.
    // 7x7, 14x14) go through the gather path, whose columns run across images
    const uint64_t hw = (uint64_t)in_h * in_w;
    const uint64_t tiles = (hw + 127) / 128;
    if (kh == 1 && kw == 1 && sh == 1 && sw == 1 && pad_top == 0 && pad_left == 0 &&
        out_h == in_h && out_w == in_w && hw <= 0x7FFFFFFFull && (tiles * 128 - hw) * 5 <= tiles * 128)
        return cm_conv_pointwise_launch(x, w, b, y, batch, in_ch, out_ch, (uint32_t)hw, epi, s);
    return cm_conv_gemm_launch(x, w, b, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                               sh, sw, dh, dw, pad_top, pad_left, epi, s);
}
