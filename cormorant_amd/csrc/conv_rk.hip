// conv_rk.hip -- small standard convolutions (any window, stride, dilation and
// padding) on int8 MFMA with the operands loaded straight into registers
// (kernels/conv/kernel/ConvKernel.cpp:171-249).
//
// y[n][m][oh][ow] = sat16(wrap32([bias[m] << 8] + sum_{c,kh_i,kw_i valid} x * w) >> 8),
// then the optional fused Add / Relu / Relu6 epilogue.
//
// The layers of a network's small feature maps (up to a few hundred thousand
// outputs; here strided windows and wide 1x1 layers, see cm_conv_rk_takes) are
// too small for the
// block-tiled kernels to fill the chip, so
// those kernels' blocks walk the whole reduction serially: 9 to 23 steps of
// 64 k for a 3x3 window over 64 to 160 channels, each step a chain of loads,
// staging and MFMAs.  Here a block of four waves owns one 32 x 32 output tile
// (32 output channels x 32 columns, a column being one output pixel of one
// image, columns running across images) and splits the reduction over its
// waves: wave w takes k steps w, w + 4, ...  Each wave loads its MFMA
// fragments straight into registers -- A, 16 consecutive k of one weight row
// (the reference order k = c * kh * kw + tap), with 16-byte loads; B, the 16
// input values of one output pixel at those k, with 2-byte loads whose
// offsets advance tap by tap -- one k step ahead of their use, splits the
// limbs in registers, and turns its accumulators into its partial sum of each
// output (mod 2^32).  The four partials meet in LDS (one barrier); each wave
// then adds, finishes and stores a quarter of the tile.  Padding taps and
// k past the end get an out-of-range buffer offset and read 0.
//
// Limbs and the exact sum are the GEMM kernel's: v = 256*vh + vl + 128 with
// vh = v >> 8, vl = (v & 255) - 128, and over the k positions a wave processes
//     sum a*b = 65536*S_hh + 256*S_mid + S_ll + 128*(sum a + sum b) - 16384*Kp
// (a zero position, limbs 0 and -128, contributes 0 to both sides), so the
// partials add up, modulo 2^32, to the whole reduction: exactly the
// accumulator's wrap.
#include "cm_internal.h"
#include "limbs.h"
#include "q88.h"

namespace {

using limbs::bsum;
using limbs::hi4;
using limbs::lo4;
using limbs::pack2;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;             // four waves: one output tile, k split four ways
constexpr uint32_t kRkMaxTaps = 32;       // window taps (a per-pixel validity bit each)
constexpr uint32_t kRkMaxSteps = 32;      // k steps of 64 (at most 8 per wave)
constexpr uint64_t kRkMaxOut = 1u << 19;  // outputs: larger layers fill the chip with the block kernels

struct RkArgs {
    const int16_t* x;
    const int16_t* w;
    const int16_t* bias;
    int16_t* y;
    EpiArgs epi;
    uint32_t C, H, W, M, OW, kh, kw, sh, sw, dh, dw, pt, pl;
    uint32_t K, kk, P, NP;        // C*kh*kw, kh*kw, OH*OW, batch*P
    uint32_t rt, nk;              // row tiles of 32, k steps of 64
    uint32_t x_bytes, w_bytes, y_bytes;
    int32_t wrap_row, wrap_c;     // element offset steps: next window row, next channel
    FastDiv div_p, div_ow, div_rt, div_kk, div_kw;
};

struct RkStep {
    uint32_t a[2][8];    // two weight rows, 16 k as packed words
    uint32_t b[2][16];   // two pixels, 16 k, one int16 per register
};

template <bool AV>
__device__ __forceinline__ void rk_load(const RkArgs& g, __amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t xr,
                                        const uint32_t (&arow)[2], const int32_t (&pbase)[2],
                                        const uint32_t (&vmask)[2], uint32_t k0, RkStep& st) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (AV) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                // K % 8 == 0: a group of 8 k values is wholly inside or outside the
                // row; an invalid row's arow is kOob, a k past the end sets bit 31
                const uint32_t hole = (uint32_t)(k0 + q * 8 >= g.K) << 31;
                const v4u v = __builtin_amdgcn_raw_buffer_load_b128(wr, (arow[i] + (k0 + q * 8) * 2u) | hole, 0, 0);
                st.a[i][4 * q + 0] = v[0]; st.a[i][4 * q + 1] = v[1];
                st.a[i][4 * q + 2] = v[2]; st.a[i][4 * q + 3] = v[3];
            }
        } else {
            uint32_t r[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t hole = (uint32_t)(k0 + e >= g.K) << 31;
                r[e] = __builtin_amdgcn_raw_buffer_load_b16(wr, (arow[i] + (k0 + e) * 2u) | hole, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) st.a[i][e] = pack2(r[2 * e], r[2 * e + 1]);
        }
    }
    // k0 -> (channel c, tap t = dy * kw + dx), then tap by tap: off is the
    // element offset of tap t of channel c from a pixel's window origin
    uint32_t c = fdiv(k0, g.div_kk), t = k0 - c * g.kk;
    uint32_t dy = fdiv(t, g.div_kw), dx = t - dy * g.kw;
    int32_t off = (int32_t)(c * g.H * g.W + dy * g.dh * g.W + dx * g.dw);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        // validity as bit 31 of the offset (past every buffer: reads 0), never as a
        // condition: the compiler turned `ok ? offset : kOob` into a branch per load
        const uint32_t kok = (uint32_t)(c < g.C);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t ok = kok & (vmask[j] >> t);
            st.b[j][e] = __builtin_amdgcn_raw_buffer_load_b16(
                xr, ((uint32_t)(pbase[j] + off) * 2u) | ((~ok & 1u) << 31), 0, 0);
        }
        // next tap, with selects: a per-lane branch here became an exec-mask
        // branch around every load
        ++t;
        ++dx;
        const bool nrow = dx == g.kw, nch = t == g.kk;
        off += (int32_t)g.dw + (nrow ? g.wrap_row : 0) + (nch ? g.wrap_c : 0);
        dx = nrow ? 0u : dx;
        t = nch ? 0u : t;
        c += nch ? 1u : 0u;
    }
}

template <bool HAS_BIAS, bool AV>
__global__ __launch_bounds__(kThreads) void conv_rk(RkArgs g) {
    __shared__ uint32_t red[kThreads / 64][16][64];   // each wave's partial sums
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t ct = fdiv(blockIdx.x, g.div_rt), rt = blockIdx.x - ct * g.rt;
    const uint32_t r16 = lane & 15, kg = lane >> 4;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(g.w, g.w_bytes), xr = make_rsrc(g.x, g.x_bytes);
    // fragment rows (output channels) and columns (image, output pixel)
    uint32_t arow[2], yoff[2], vmask[2];
    int32_t pbase[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t m = rt * 32u + i * 16u + r16;
        arow[i] = m < g.M ? m * g.K * 2u : kOob;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t col = ct * 32u + j * 16u + r16;
        const uint32_t n = fdiv(col, g.div_p), p = col - n * g.P;
        const uint32_t oh = fdiv(p, g.div_ow), ow = p - oh * g.OW;
        const int32_t ih0 = (int32_t)(oh * g.sh) - (int32_t)g.pt, iw0 = (int32_t)(ow * g.sw) - (int32_t)g.pl;
        pbase[j] = (int32_t)(n * g.C * g.H * g.W) + ih0 * (int32_t)g.W + iw0;
        uint32_t vm = 0;
        for (uint32_t dy = 0; dy < g.kh; ++dy) {
            const bool rok = (uint32_t)(ih0 + (int32_t)(dy * g.dh)) < g.H;
            for (uint32_t dx = 0; dx < g.kw; ++dx)
                if (rok && (uint32_t)(iw0 + (int32_t)(dx * g.dw)) < g.W) vm |= 1u << (dy * g.kw + dx);
        }
        vmask[j] = col < g.NP ? vm : 0u;
        yoff[j] = col < g.NP ? n * g.M * g.P + p : 0xFFFFFFFFu;
    }
    // this wave finishes outputs v = 4 * wave + u (u = 0..3) of the lane's 16:
    // row tile i = wave >> 1, rows 4 * kg + e with e = 2 * (wave & 1) + (u >> 1),
    // column j = u & 1; their bias and fused-Add operands load now, behind the k loop
    const uint32_t fi = wave >> 1;
    uint32_t fbias[2] = {0u, 0u}, fadd[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t m = rt * 32u + fi * 16u + kg * 4u + 2u * (wave & 1u) + (uint32_t)h;
        if constexpr (HAS_BIAS) fbias[h] = q88::data_to_acc(g.bias[m < g.M ? m : 0u]);
        if (g.epi.add_mode == 1u) {
            const __amdgpu_buffer_rsrc_t ar = make_rsrc(g.epi.add, g.y_bytes);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const bool ok = m < g.M && yoff[j] != 0xFFFFFFFFu;
                fadd[2 * h + j] = __builtin_amdgcn_raw_buffer_load_b16(ar, ok ? (yoff[j] + m * g.P) * 2u : kOob, 0, 0);
            }
        }
    }

    v4i hh[2][2], mid[2][2], ll[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) hh[i][j] = mid[i][j] = ll[i][j] = v4i{0, 0, 0, 0};
    int32_t ahs[2] = {0, 0}, als[2] = {0, 0}, bhs[2] = {0, 0}, bls[2] = {0, 0};
    auto compute = [&](const RkStep& st) {
        v4i ah[2], al[2], bh[2], bl[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t h = hi4(st.a[i][2 * q], st.a[i][2 * q + 1]);
                const uint32_t l = lo4(st.a[i][2 * q], st.a[i][2 * q + 1]);
                ah[i][q] = (int)h; al[i][q] = (int)l;
                ahs[i] = bsum(h, ahs[i]); als[i] = bsum(l, als[i]);
            }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t w0 = pack2(st.b[j][4 * q], st.b[j][4 * q + 1]);
                const uint32_t w1 = pack2(st.b[j][4 * q + 2], st.b[j][4 * q + 3]);
                const uint32_t h = hi4(w0, w1), l = lo4(w0, w1);
                bh[j][q] = (int)h; bl[j][q] = (int)l;
                bhs[j] = bsum(h, bhs[j]); bls[j] = bsum(l, bls[j]);
            }
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                hh[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bh[j], hh[i][j], 0, 0, 0);
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bl[j], mid[i][j], 0, 0, 0);
                ll[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bl[j], ll[i][j], 0, 0, 0);
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bh[j], mid[i][j], 0, 0, 0);
            }
    };
    // this wave's steps: s = wave, wave + 4, ... (two register stages; past the
    // last step the loads read 0 through kOob and are never used)
    const uint32_t kl = kg * 16u;
    uint32_t my = 0;
    RkStep s0, s1;
    rk_load<AV>(g, wr, xr, arow, pbase, vmask, wave * 64u + kl, s0);
    for (uint32_t s = wave; s < g.nk; s += 8) {
        rk_load<AV>(g, wr, xr, arow, pbase, vmask, (s + 4) * 64u + kl, s1);
        compute(s0);
        ++my;
        if (s + 4 >= g.nk) break;
        rk_load<AV>(g, wr, xr, arow, pbase, vmask, (s + 8) * 64u + kl, s0);
        compute(s1);
        ++my;
    }

    // the wave's partial sum of each of the lane's 16 outputs (mod 2^32)
    const uint32_t kp = my * 64u;
    uint32_t rsum[2], csum[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint32_t v = 256u * (uint32_t)ahs[i] + (uint32_t)als[i];
        v += (uint32_t)__shfl_xor((int)v, 16, 64);
        v += (uint32_t)__shfl_xor((int)v, 32, 64);
        rsum[i] = v + 128u * kp;
        uint32_t u = 256u * (uint32_t)bhs[i] + (uint32_t)bls[i];
        u += (uint32_t)__shfl_xor((int)u, 16, 64);
        u += (uint32_t)__shfl_xor((int)u, 32, 64);
        csum[i] = u + 128u * kp;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t rs = (uint32_t)__shfl((int)rsum[i], (int)(kg * 4u + (uint32_t)e), 64);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                red[wave][i * 8 + e * 2 + j][lane] =
                    65536u * (uint32_t)hh[i][j][e] + 256u * (uint32_t)mid[i][j][e] + (uint32_t)ll[i][j][e] +
                    128u * (rs + csum[j]) - 16384u * kp;
        }
    __syncthreads();
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t e = 2u * (wave & 1u) + (uint32_t)h;
        const uint32_t m = rt * 32u + fi * 16u + kg * 4u + e;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t v = fi * 8u + e * 2u + (uint32_t)j;
            const uint32_t acc = red[0][v][lane] + red[1][v][lane] + red[2][v][lane] + red[3][v][lane] + fbias[h];
            if (m >= g.M || yoff[j] == 0xFFFFFFFFu) continue;
            int32_t o = q88::acc_to_data(acc);
            if (g.epi.add_mode == 1u) o = q88::add(o, (int16_t)fadd[2 * h + j]);
            g.y[yoff[j] + m * g.P] = (int16_t)q88::clamp(o, lo, hi);
        }
    }
}

}  // namespace

// The shapes this path takes (a pure function of the shape, so that the packed
// weight query can mirror the dispatch).
bool cm_conv_rk_takes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                      uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t sh, uint32_t sw,
                      uint32_t dh, uint32_t dw, uint32_t pad_top, uint32_t pad_left) {
    const uint64_t kk = (uint64_t)kh * kw, K = (uint64_t)in_ch * kk;
    const uint64_t np = (uint64_t)batch * out_h * out_w;
    if (kk > kRkMaxTaps || in_ch == 0 || out_ch == 0 || np == 0) return false;
    // Strided windows, and 1x1 convolutions (stride 1, no padding) over at least
    // 128 channels.  Measured on MobileNetV2-like layers (batch 16): 3x3 stride 2
    // at 28x28 / 14x14 / 7x7 outputs took 8.5 / 9.1 / 12.3 us here against 10.2 /
    // 10.6 / 14.6 on the patch GEMM, while stride-1 3x3 layers tied (64 and 160
    // channels) or lost (96 channels at 14x14: 17.3 against 14.5 us): a wave holds
    // one k step of loads in flight, and each step waits ~1.5 us for them.  A 1x1
    // layer gathers nothing twice, and splitting its k steps over four waves
    // shortens the chain the one-wave-per-tile 1x1 kernel walks: 160 -> 160 / 320
    // at 7x7 5.4 / 5.6 us against 7.9 / 8.1, 1280 -> 256 12.7 us against 36 on the
    // gather GEMM (past that kernel's 512 channels); below 128 channels it tied.
    if (kk == 1) {
        if (sh != 1 || sw != 1 || pad_top != 0 || pad_left != 0 || in_ch < 128) return false;
    } else if (sh * sw < 2) {
        return false;
    }
    if ((K + 63) / 64 > kRkMaxSteps || (uint64_t)out_ch * np > kRkMaxOut) return false;
    const uint64_t x_bytes = 2ull * batch * in_ch * in_h * in_w;
    if (x_bytes >= 0x80000000ull || 2ull * out_ch * K >= 0x80000000ull) return false;
    // window offsets in int32: planes, strides, dilations and pads below 2^15
    return in_h < (1u << 15) && in_w < (1u << 15) &&
           (uint64_t)out_h * sh + (uint64_t)kh * dh + pad_top < (1u << 15) &&
           (uint64_t)out_w * sw + (uint64_t)kw * dw + pad_left < (1u << 15);
}

int cm_conv_rk_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y, uint32_t batch,
                      uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h,
                      uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t sh, uint32_t sw, uint32_t dh,
                      uint32_t dw, uint32_t pad_top, uint32_t pad_left, const cm_epilogue_t* epi,
                      const LaunchCtx& lc) {
    if (!cm_conv_rk_takes(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top,
                          pad_left))
        return 1;
    if (lc.need) return CM_OK;   // no workspace
    RkArgs g{};
    g.x = x; g.w = w; g.bias = bias; g.y = y; g.epi = cm_epi_args(epi);
    g.C = in_ch; g.H = in_h; g.W = in_w; g.M = out_ch; g.OW = out_w;
    g.kh = kh; g.kw = kw; g.sh = sh; g.sw = sw; g.dh = dh; g.dw = dw; g.pt = pad_top; g.pl = pad_left;
    g.kk = kh * kw;
    g.K = in_ch * g.kk;
    g.P = out_h * out_w;
    g.NP = batch * g.P;
    g.rt = (out_ch + 31) / 32;
    g.nk = (g.K + 63) / 64;
    g.x_bytes = (uint32_t)(2ull * batch * in_ch * in_h * in_w);
    g.w_bytes = (uint32_t)(2ull * out_ch * g.K);
    g.y_bytes = (uint32_t)(2ull * out_ch * g.NP);
    g.wrap_row = (int32_t)(dh * in_w) - (int32_t)(kw * dw);
    g.wrap_c = (int32_t)(in_h * in_w) - (int32_t)(kh * dh * in_w);
    g.div_p = make_fastdiv(g.P);
    g.div_ow = make_fastdiv(out_w);
    g.div_rt = make_fastdiv(g.rt);
    g.div_kk = make_fastdiv(g.kk);
    g.div_kw = make_fastdiv(kw);
    const uint64_t blocks = (uint64_t)g.rt * ((g.NP + 31) / 32);
    const dim3 grid((uint32_t)blocks);
    const bool av = g.K % 8 == 0 && ((uintptr_t)w & 15u) == 0;
    if (bias) {
        if (av) hipLaunchKernelGGL((conv_rk<true, true>), grid, dim3(kThreads), 0, lc.s, g);
        else hipLaunchKernelGGL((conv_rk<true, false>), grid, dim3(kThreads), 0, lc.s, g);
    } else {
        if (av) hipLaunchKernelGGL((conv_rk<false, true>), grid, dim3(kThreads), 0, lc.s, g);
        else hipLaunchKernelGGL((conv_rk<false, false>), grid, dim3(kThreads), 0, lc.s, g);
    }
    return cm_check_launch("conv_rk");
}
