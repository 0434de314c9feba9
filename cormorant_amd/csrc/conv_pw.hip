// conv_pw.hip -- small pointwise convolutions (1x1, stride 1, no padding) on
// int8 MFMA with no LDS and no barrier (kernels/conv/kernel/ConvKernel.cpp:171-249).
//
// y[n][m][p] = sat16(wrap32([bias[m] << 8] + sum_c w[m][c] * x[n][c][p]) >> 8),
// then the optional fused Add / Relu / Relu6 epilogue.
//
// For the small layers of a network (a few hundred thousand outputs, K <= 512)
// the block-tiled GEMM spends most of its time in a chain of dependent phases:
// global loads, limb split into LDS, barrier, fragment reads, MFMAs, an LDS
// epilogue tile, barrier, stores.  Here each wave owns one 32 x 32 output tile
// (32 output channels x 32 columns, a column being one pixel of one image,
// columns running across images) and loads its MFMA fragments straight into
// registers: the A fragment (16 consecutive k of one weight row) with 16-byte
// loads, the B fragment (16 channels of one pixel, P elements apart) with
// 2-byte loads.  Every load is a range-checked buffer load (an invalid row,
// column or k reads 0) issued one k step ahead of its use; the limbs are split
// in registers and the sums leave the accumulators directly.
//
// Limbs and the exact sum are the GEMM kernel's: v = 256*vh + vl + 128 with
// vh = v >> 8, vl = (v & 255) - 128, and
//     sum a*b = 65536*S_hh + 256*S_mid + S_ll + 128*(sum a + sum b) - 16384*Kp
// over Kp = 64 * steps k positions (a zero-padded position, whose limbs are
// 0 and -128, contributes 0 to both sides).  Every term is taken modulo 2^32,
// the accumulator's own wrap.  |S_mid| stays below 2^31 for K <= 2^15.
#include "cm_internal.h"
#include "limbs.h"
#include "q88.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;            // four independent waves
constexpr uint32_t kPwMaxK = 512;        // in_ch limit of this path
constexpr uint64_t kPwMaxOut = 1u << 21; // outputs limit of this path (larger layers fill the
                                         // chip with the block-tiled GEMM)

struct PwArgs {
    const int16_t* x;
    const int16_t* w;
    const int16_t* bias;
    int16_t* y;
    EpiArgs epi;
    uint32_t C, M, P, NP;   // in_ch, out_ch, pixels per image, columns (images * P)
    uint32_t rt, nk;        // row tiles of 32; k steps of 64
    uint32_t x_bytes, w_bytes, y_bytes;
    FastDiv div_p, div_rt;
    // GAP form: row-tile pairs per image, and 1 / P for the average's finaliser
    uint32_t rtp;
    float inv_p;
};

using limbs::hi4;
using limbs::lo4;
using limbs::bsum;
using limbs::pack2;

// One k step's raw operands of a lane: 16 k values of its two weight rows (as
// 8 packed words each) and of its two columns (one int16 per register).
struct PwStep {
    uint32_t a[2][8];
    uint32_t b[2][16];
};

template <bool AV>
__device__ __forceinline__ void pw_load(const PwArgs& g, __amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t xr,
                                        const uint32_t (&arow)[2], const uint32_t (&bcol)[2], uint32_t kb,
                                        PwStep& st) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (AV) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                // C % 8 == 0: a group of 8 k values is wholly inside or outside the
                // row; an invalid row's arow is kOob, a k past the end sets bit 31
                // (validity in the offset: a select on it became a branch per load)
                const uint32_t hole = (uint32_t)(kb + q * 8 >= g.C) << 31;
                const v4u v = __builtin_amdgcn_raw_buffer_load_b128(wr, (arow[i] + (kb + q * 8) * 2u) | hole, 0, 0);
                st.a[i][4 * q + 0] = v[0]; st.a[i][4 * q + 1] = v[1];
                st.a[i][4 * q + 2] = v[2]; st.a[i][4 * q + 3] = v[3];
            }
        } else {
            uint32_t r[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t hole = (uint32_t)(kb + e >= g.C) << 31;
                r[e] = __builtin_amdgcn_raw_buffer_load_b16(wr, (arow[i] + (kb + e) * 2u) | hole, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) st.a[i][e] = pack2(r[2 * e], r[2 * e + 1]);
        }
    }
    const uint32_t cst = g.P * 2u;   // bytes between two channels of one pixel
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            // an invalid column's bcol is kOob (the sum stays below 2^32)
            const uint32_t hole = (uint32_t)(kb + e >= g.C) << 31;
            st.b[j][e] = __builtin_amdgcn_raw_buffer_load_b16(xr, (bcol[j] + (kb + e) * cst) | hole, 0, 0);
        }
}

// GAP: the convolution followed by GlobalAveragePool of every output plane
// (P <= 64), y = [image][channel].  A block is one image and two 32-channel row
// tiles; its waves 2t and 2t + 1 take row tile t's pixels 0-31 and 32-63 (the
// columns past P read 0 and are left out of the sums), each sums its finished
// outputs (sat16, activation: the values the unfused convolution would store)
// over its pixels as the pool's accumulator does (value << 8, mod 2^32), the
// two halves meet in LDS, and the even wave finishes the average
// (PoolingKernel.cpp:253-266 through the pool kernels' own finaliser).
template <bool HAS_BIAS, bool AV, bool GAP>
__global__ __launch_bounds__(kThreads) void conv_pw(PwArgs g) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    uint32_t ct, rt, gap_n = 0, half = 0;
    if constexpr (GAP) {
        gap_n = blockIdx.x / g.rtp;
        rt = (blockIdx.x - gap_n * g.rtp) * 2u + (wave >> 1);
        half = wave & 1u;
        ct = 0;
    } else {
        const uint32_t wid = blockIdx.x * (kThreads / 64) + wave;
        ct = fdiv(wid, g.div_rt);
        rt = wid - ct * g.rt;   // waves of a block share columns
        if (ct * 32u >= g.NP) return;   // the whole wave
    }
    const uint32_t r16 = lane & 15, kg = lane >> 4;
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(g.w, g.w_bytes), xr = make_rsrc(g.x, g.x_bytes);
    // this lane's fragment rows (output channels) and columns (image, pixel)
    uint32_t arow[2], bcol[2], yoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t m = rt * 32u + i * 16u + r16;
        arow[i] = m < g.M ? m * g.C * 2u : kOob;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        if constexpr (GAP) {
            const uint32_t p = half * 32u + j * 16u + r16;
            bcol[j] = p < g.P ? (gap_n * g.C * g.P + p) * 2u : kOob;
            yoff[j] = p < g.P ? 0u : 0xFFFFFFFFu;
        } else {
            const uint32_t col = ct * 32u + j * 16u + r16;
            const uint32_t n = fdiv(col, g.div_p), p = col - n * g.P;
            bcol[j] = col < g.NP ? (n * g.C * g.P + p) * 2u : kOob;
            yoff[j] = col < g.NP ? n * g.M * g.P + p : 0xFFFFFFFFu;
        }
    }
    // the bias and the fused Add's operand of every output this lane stores,
    // loaded now so that their latency hides behind the k loop (loaded in the
    // epilogue they added a memory round trip to every launch: ~1.6 us)
    uint32_t addv[2][4][2], biasv[2][4];
    if constexpr (HAS_BIAS) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = rt * 32u + i * 16u + kg * 4u + (uint32_t)e;
                biasv[i][e] = q88::data_to_acc(g.bias[m < g.M ? m : 0u]);
            }
    }
    if (!GAP && g.epi.add_mode == 1u) {
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(g.epi.add, g.y_bytes);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t m = rt * 32u + i * 16u + kg * 4u + (uint32_t)e;
                    const bool ok = m < g.M && yoff[j] != 0xFFFFFFFFu;
                    addv[i][e][j] = __builtin_amdgcn_raw_buffer_load_b16(ar, ok ? (yoff[j] + m * g.P) * 2u : kOob, 0, 0);
                }
    }
    v4i hh[2][2], mid[2][2], ll[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) hh[i][j] = mid[i][j] = ll[i][j] = v4i{0, 0, 0, 0};
    int32_t ahs[2] = {0, 0}, als[2] = {0, 0}, bhs[2] = {0, 0}, bls[2] = {0, 0};

    auto compute = [&](const PwStep& st) {
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
    // two register stages: step s + 1 loads while step s computes (past the last
    // step the loads read 0 through kOob and are never used)
    PwStep s0, s1;
    pw_load<AV>(g, wr, xr, arow, bcol, kg * 16u, s0);
    for (uint32_t s = 0; s < g.nk; s += 2) {
        pw_load<AV>(g, wr, xr, arow, bcol, (s + 1) * 64u + kg * 16u, s1);
        compute(s0);
        if (s + 1 >= g.nk) break;
        pw_load<AV>(g, wr, xr, arow, bcol, (s + 2) * 64u + kg * 16u, s0);
        compute(s1);
    }

    // sums over all k of each fragment row / column: the four k groups of a row
    // are lanes l, l ^ 16, l ^ 32, l ^ 48 (sum a = 256 * hs + ls + 128 * count)
    const uint32_t kp = g.nk * 64u;
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
    // epilogue: lane holds rows 4 * kg + e (e = 0..3) of each 16-row tile, column r16
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    uint32_t gsum[2][4] = {};   // GAP: this lane's columns' (value << 8) per row
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t rr = kg * 4u + (uint32_t)e;
            const uint32_t rs = (uint32_t)__shfl((int)rsum[i], (int)rr, 64);
            const uint32_t m = rt * 32u + i * 16u + rr;
            if (m >= g.M) continue;
            const uint32_t b8 = HAS_BIAS ? biasv[i][e] : 0u;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (yoff[j] == 0xFFFFFFFFu) continue;
                const uint32_t acc = 65536u * (uint32_t)hh[i][j][e] + 256u * (uint32_t)mid[i][j][e] +
                                     (uint32_t)ll[i][j][e] + 128u * (rs + csum[j]) - 16384u * kp + b8;
                int32_t v = q88::acc_to_data(acc);
                if constexpr (GAP) {
                    gsum[i][e] += (uint32_t)q88::clamp(v, lo, hi) << 8;
                } else {
                    const uint32_t yi = yoff[j] + m * g.P;
                    if (g.epi.add_mode == 1u) v = q88::add(v, (int16_t)addv[i][e][j]);
                    g.y[yi] = (int16_t)q88::clamp(v, lo, hi);
                }
            }
        }
    if constexpr (GAP) {
        // the sixteen columns of a row are the lanes of one 16-lane group
        __shared__ uint32_t part[kThreads / 64][32];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t v = gsum[i][e];
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
                if (r16 == 0) part[wave][i * 16 + kg * 4 + e] = v;
            }
        __syncthreads();
        if (half == 0 && lane < 32u) {
            const uint32_t m = rt * 32u + lane;
            if (m < g.M)
                g.y[(uint64_t)gap_n * g.M + m] = q88::avg_finalize(part[wave][lane] + part[wave + 1][lane], g.inv_p);
        }
    }
}

}  // namespace

// Returns 1 when the shape is not for this path (the caller tries another).
int cm_conv_pw_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                      uint32_t batch, uint32_t in_ch, uint32_t out_ch, uint32_t hw,
                      const cm_epilogue_t* epi, const LaunchCtx& lc) {
    const uint64_t np = (uint64_t)batch * hw;
    if (in_ch == 0 || in_ch > kPwMaxK || np == 0 || out_ch == 0) return 1;
    if ((uint64_t)out_ch * np > kPwMaxOut) return 1;
    const uint64_t x_bytes = 2ull * in_ch * np, w_bytes = 2ull * out_ch * in_ch;
    const uint64_t y_elems = (uint64_t)out_ch * np;
    if (x_bytes >= 0x80000000ull || w_bytes >= 0x80000000ull || y_elems >= 0xFFFFFFFFull) return 1;
    if (lc.need) return CM_OK;   // no workspace
    const EpiArgs ea = cm_epi_args(epi);
    PwArgs g{};
    g.x = x; g.w = w; g.bias = bias; g.y = y; g.epi = ea;
    g.C = in_ch; g.M = out_ch; g.P = hw; g.NP = (uint32_t)np;
    g.rt = (out_ch + 31) / 32;
    g.nk = (in_ch + 63) / 64;
    g.x_bytes = (uint32_t)x_bytes; g.w_bytes = (uint32_t)w_bytes; g.y_bytes = (uint32_t)(2 * y_elems);
    g.div_p = make_fastdiv(hw);
    g.div_rt = make_fastdiv(g.rt);
    const uint64_t waves = (uint64_t)g.rt * ((np + 31) / 32);
    const dim3 grid((uint32_t)((waves + 3) / 4));
    const bool av = in_ch % 8 == 0 && ((uintptr_t)w & 15u) == 0;
    if (bias) {
        if (av) hipLaunchKernelGGL((conv_pw<true, true, false>), grid, dim3(kThreads), 0, lc.s, g);
        else hipLaunchKernelGGL((conv_pw<true, false, false>), grid, dim3(kThreads), 0, lc.s, g);
    } else {
        if (av) hipLaunchKernelGGL((conv_pw<false, true, false>), grid, dim3(kThreads), 0, lc.s, g);
        else hipLaunchKernelGGL((conv_pw<false, false, false>), grid, dim3(kThreads), 0, lc.s, g);
    }
    return cm_check_launch("conv_pw");
}

// The 1x1 convolution + activation + GlobalAveragePool shapes cm_conv_gap runs:
// planes of at most 64 pixels, the register-only kernel's channel limit, and
// operands whose byte offsets fit the buffer ranges.
bool cm_conv_gap_fits(uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch) {
    if (batch == 0 || in_ch == 0 || in_ch > kPwMaxK || hw == 0 || hw > 64 || out_ch == 0) return false;
    const uint64_t x_bytes = 2ull * in_ch * hw * batch, w_bytes = 2ull * out_ch * in_ch;
    const uint64_t blocks = (uint64_t)batch * ((out_ch + 63) / 64);
    return x_bytes < 0x80000000ull && w_bytes < 0x80000000ull && blocks < 0x80000000ull &&
           (uint64_t)batch * out_ch < 0xFFFFFFFFull;
}

int cm_conv_gap_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                       uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch, uint32_t act,
                       hipStream_t s) {
    PwArgs g{};
    g.x = x; g.w = w; g.bias = bias; g.y = y;
    g.epi = EpiArgs{};
    g.epi.act = act;
    g.C = in_ch; g.M = out_ch; g.P = hw; g.NP = batch * hw;
    g.rt = (out_ch + 31) / 32;
    g.rtp = (g.rt + 1) / 2;
    g.nk = (in_ch + 63) / 64;
    g.x_bytes = 2u * in_ch * hw * batch; g.w_bytes = 2u * out_ch * in_ch; g.y_bytes = 2u * batch * out_ch;
    g.div_p = make_fastdiv(hw);
    g.div_rt = make_fastdiv(g.rt);
    g.inv_p = 1.0f / (float)hw;
    const dim3 grid(batch * g.rtp);
    const bool av = in_ch % 8 == 0 && ((uintptr_t)w & 15u) == 0;
    if (bias) {
        if (av) hipLaunchKernelGGL((conv_pw<true, true, true>), grid, dim3(kThreads), 0, s, g);
        else hipLaunchKernelGGL((conv_pw<true, false, true>), grid, dim3(kThreads), 0, s, g);
    } else {
        if (av) hipLaunchKernelGGL((conv_pw<false, true, true>), grid, dim3(kThreads), 0, s, g);
        else hipLaunchKernelGGL((conv_pw<false, false, true>), grid, dim3(kThreads), 0, s, g);
    }
    return cm_check_launch("conv_gap");
}
