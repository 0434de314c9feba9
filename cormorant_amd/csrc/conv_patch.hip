// conv_patch.hip -- 3x3 convolution (stride 1 or 2, dilation 1) with few
// channels on int8 MFMA, from an input patch staged once per output tile.
//
// Reference arithmetic (kernels/conv/kernel/ConvKernel.cpp:160-169, 231-249,
// 333): acc = wrap32([bias << 8] + sum_{c,kh,kw} x * w), out = sat16(acc >> 8),
// with padded taps skipped (they hold 0 here, which adds nothing).
//
// The implicit-GEMM path gathers every (k, pixel) element of its B tile with a
// 2-byte load, nine times per input value for a 3x3 window.  Here a block owns
// an output tile of 8 rows x 16 columns of one image and all (<= 64) output
// channels; it loads the tile's input patch ((7S+3) x (15S+3) positions, every
// channel) once, and stores it in LDS channel-minor as int8 limbs: position p,
// channel c at byte p * ppitch + c of a high-byte plane and a low-byte plane.
// With the reduction index ordered k = tap * C16 + c (C16 = channels rounded
// up to 16), the 16 k values an MFMA lane supplies are 16 channels of one tap
// at one position: one 16-byte LDS read, so the B operand needs no staging per
// k step.  The weights are staged once per block in the same k order.  The
// row and column sums the identity needs are taken (v_dot4 with ones) from the
// very operand registers the MFMAs consume, next to them in the k loop.
//
// Limbs and the exact sum are those of the GEMM kernel: v = 256*vh + vl + 128
// with vh = v >> 8, vl = (v & 255) - 128, and
//   sum a*b = 65536*S_hh + 256*S_mid + S_ll + 128*(sum a + sum b) - 16384*Kp
// over Kp = nk * 64 k positions; a position with a zero operand (padding
// channels, taps outside the image, k past 9*C16) contributes 0 to both sides.
// Every term is taken modulo 2^32, the accumulator's wrap.
#include "cm_internal.h"
#include "q88.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v2s __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int TH = 8, TW = 16, TP = TH * TW;   // output tile: 8 rows x 16 columns
constexpr int kTilePitch = TP + 4;             // epilogue tile: uint32 per row
constexpr int kAB = 6;                         // weight vectors in flight per thread
constexpr int kPB = 6;                         // patch tasks (4 loads each) in flight per thread

struct PatchArgs {
    const int16_t* x;
    const int16_t* w;
    const int16_t* bias;
    int16_t* y;
    uint32_t C, H, W, M, OH, OW, pt, pl;
    uint32_t C16, nk;            // channels rounded up to 16; k steps of 64 covering 9*C16
    uint32_t apitch, ppitch;     // LDS bytes per weight row / per patch position
    uint32_t p_off;              // LDS byte offset of the patch planes
    uint32_t tiles_w, tiles_h;
    FastDiv div_tw, div_th, div_k;
    uint32_t x_img_bytes;        // one image of x, < 2^31
    uint64_t x_img, y_img;       // elements per image
    uint32_t vw;                 // output / Add access width in elements (8, 4, 2 or 1)
    EpiArgs epi;
};

template <int S>
struct PatchGeom {
    static constexpr int PR = (TH - 1) * S + 3, PW = (TW - 1) * S + 3, NPOS = PR * PW;
};

__device__ __forceinline__ uint32_t hi_byte(int32_t v) { return (uint32_t)(v >> 8) & 0xFFu; }
__device__ __forceinline__ uint32_t lo_byte(int32_t v) { return ((uint32_t)v & 0xFFu) ^ 0x80u; }
// sum of the 16 signed bytes of v, added to acc
__device__ __forceinline__ int32_t bsum16(v4i v, int32_t acc) {
#pragma unroll
    for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_sdot4(v[q], 0x01010101, acc, false);
    return acc;
}

template <int MT, int S, bool HAS_BIAS>
// at most 128 registers (with the accumulators) for 4 resident blocks per CU
// where MT <= 32; MT = 64 keeps its accumulators at 2 blocks per CU
__global__ __launch_bounds__(kThreads, MT <= 32 ? 4 : 2) void conv_patch(PatchArgs g) {
    using PG = PatchGeom<S>;
    constexpr int PW = PG::PW, NPOS = PG::NPOS;
    constexpr int MI = MT / 16;   // MFMA row tiles
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t colsum[TP], rowsum[MT], biasv[MT];
    uint8_t* a_hi = lds;
    uint8_t* a_lo = lds + MT * g.apitch;
    uint8_t* p_hi = lds + g.p_off;
    uint8_t* p_lo = p_hi + NPOS * g.ppitch;
    uint32_t* tile = reinterpret_cast<uint32_t*>(lds);   // epilogue, after the MFMA phase

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t tq = fdiv(blockIdx.x, g.div_tw), tw = blockIdx.x - tq * g.tiles_w;
    const uint32_t n = fdiv(tq, g.div_th), th = tq - n * g.tiles_h;
    const uint32_t oh0 = th * TH, ow0 = tw * TW;
    const int32_t ih0 = (int32_t)(oh0 * S) - (int32_t)g.pt;
    const int32_t iw0 = (int32_t)(ow0 * S) - (int32_t)g.pl;
    const uint32_t K = g.C * 9;
    const uint32_t Q = 9 * g.C16 / 16;   // chunks holding real taps
    const uint32_t cpt = g.C16 / 16;     // chunks per tap


    // Weight limb planes: row m, byte (tap * C16 + c).  They start as the
    // encoding of 0 (high 0, low 0x80), which padding channels, k past 9*C16
    // and rows past M keep.
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(g.w, g.M * K * 2u);
    const uint32_t nvec = g.M * K / 8;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(g.x + (uint64_t)n * g.x_img, g.x_img_bytes);
    const uint32_t hw = g.H * g.W;
    const uint32_t ntask = (g.C16 / 4) * NPOS;   // (4 channels, position) pairs of the patch

    // Patch: task e = (channel group c4, position pos), pos fastest so the
    // lanes of a load read neighbouring columns; positions outside the image
    // and channels past C read 0 through the buffer range.
    auto patch_issue = [&](uint32_t b0, uint32_t (&v)[kPB][4]) {
#pragma unroll
        for (int u = 0; u < kPB; ++u) {
            const uint32_t e = b0 + u * kThreads + tid;
            const uint32_t c4 = e / NPOS, pos = e - c4 * NPOS;
            const uint32_t r = pos / PW, col = pos - r * PW;
            const int32_t ih = ih0 + (int32_t)r, iw = iw0 + (int32_t)col;
            // validity as bits, and an invalid offset made out of range by its
            // bit 31: a condition here would become a branch around the load,
            // and the compiler then waits for every load at the merge
            const uint32_t okp = (uint32_t)(e < ntask) & (uint32_t)((uint32_t)ih < g.H) &
                                 (uint32_t)((uint32_t)iw < g.W);
            const uint32_t base = ((c4 * 4) * hw + (uint32_t)ih * g.W + (uint32_t)iw) * 2u;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t okc = okp & (uint32_t)(c4 * 4 + j < g.C);
                const uint32_t off = ((base + j * hw * 2u) & 0x7FFFFFFFu) | ((okc ^ 1u) << 31);
                v[u][j] = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(xrs, off, 0, 0);
            }
        }
    };
    // limb words of 4 channels at one position
    auto patch_store = [&](uint32_t b0, const uint32_t (&v)[kPB][4]) {
#pragma unroll
        for (int u = 0; u < kPB; ++u) {
            const uint32_t e = b0 + u * kThreads + tid;
            if (e < ntask) {
                const uint32_t c4 = e / NPOS, pos = e - c4 * NPOS;
                uint32_t wh = 0, wl = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int32_t x = (int32_t)(int16_t)v[u][j];
                    wh |= hi_byte(x) << (8 * j);
                    wl |= lo_byte(x) << (8 * j);
                }
                *reinterpret_cast<uint32_t*>(p_hi + pos * g.ppitch + c4 * 4) = wh;
                *reinterpret_cast<uint32_t*>(p_lo + pos * g.ppitch + c4 * 4) = wl;
            }
        }
    };

    // Weights (nvec >= 9: the host requires C % 8 == 0, so K >= 72): 16-byte
    // loads of batch b0, then each value's two limb bytes to its place.
    auto w_issue = [&](uint32_t b0, v4u (&v)[kAB]) {
#pragma unroll
        for (int u = 0; u < kAB; ++u) {
            const uint32_t idx = b0 + u * kThreads + tid;
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(wrs, idx < nvec ? idx * 16u : kOob, 0, 0);
        }
    };
    auto w_store = [&](uint32_t b0, const v4u (&v)[kAB]) {
#pragma unroll
        for (int u = 0; u < kAB; ++u) {
            const uint32_t idx = b0 + u * kThreads + tid;
            if (idx < nvec) {
                const uint32_t e = idx * 8;
                const uint32_t m = fdiv(e, g.div_k), k = e - m * K;
                const v8s sv = __builtin_bit_cast(v8s, v[u]);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t c = (k + j) / 9, tap = (k + j) - c * 9;
                    const uint32_t d = m * g.apitch + tap * g.C16 + c;
                    a_hi[d] = (uint8_t)hi_byte(sv[j]);
                    a_lo[d] = (uint8_t)lo_byte(sv[j]);
                }
            }
        }
    };

    // The first batches of weight and patch loads (all of them for most
    // layers) are issued back to back, outside any loop: a loop entered with
    // loads in flight whose values it does not use makes the compiler wait
    // for them first.  The bias is loaded here and used only at the end.
    // The weight planes are cleared while the loads fly.
    uint32_t bias_raw = 0;
    if constexpr (HAS_BIAS) {   // a buffer load (threads past M read 0): no branch around it
        const __amdgpu_buffer_rsrc_t brs = make_rsrc(g.bias, g.M * 2u);
        bias_raw = (uint32_t)(int32_t)(int16_t)__builtin_amdgcn_raw_buffer_load_b16(
            brs, tid < g.M ? tid * 2u : kOob, 0, 0);
    }
    v4u wv[kAB];
    uint32_t pv[kPB][4];
    w_issue(0, wv);
    patch_issue(0, pv);
    {
        uint32_t* ah = reinterpret_cast<uint32_t*>(a_hi);
        uint32_t* al = reinterpret_cast<uint32_t*>(a_lo);
        const uint32_t nw = MT * g.apitch / 4;
        for (uint32_t i = tid; i < nw; i += kThreads) { ah[i] = 0u; al[i] = 0x80808080u; }
    }
    __syncthreads();
    w_store(0, wv);
    patch_store(0, pv);
    for (uint32_t b0 = kThreads * kAB; b0 < nvec; b0 += kThreads * kAB) {
        w_issue(b0, wv);
        w_store(b0, wv);
    }
    for (uint32_t b0 = kThreads * kPB; b0 < ntask; b0 += kThreads * kPB) {
        patch_issue(b0, pv);
        patch_store(b0, pv);
    }
    if (HAS_BIAS && tid < MT) biasv[tid] = bias_raw * 256u;
    __syncthreads();

    // MFMA phase: wave w owns tile rows 2w, 2w+1 (16 columns each) and all MT
    // output channels.
    v4i hh[MI][2], mid[MI][2], ll[MI][2];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            hh[i][j] = v4i{0, 0, 0, 0}; mid[i][j] = v4i{0, 0, 0, 0}; ll[i][j] = v4i{0, 0, 0, 0};
        }
    uint32_t bbase[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) bbase[j] = ((wave * 2 + j) * S * PW + (lane & 15) * S) * g.ppitch;
    const uint32_t qin = lane >> 4;
    // limb sums of this lane's A rows / B columns over its k chunks
    int32_t rh[MI], rl[MI], ch[2] = {0, 0}, cl[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < MI; ++i) { rh[i] = 0; rl[i] = 0; }
    // chunk q = tap * cpt + c0 / 16: its offset from the column's window origin,
    // in registers (tap = q / cpt by a multiply: exact for q < 36, cpt <= 4)
    const uint32_t m_cpt = (256u + cpt - 1u) / cpt;
    for (uint32_t it = 0; it < g.nk; ++it) {
        const uint32_t q = it * 4 + qin;
        const bool real = q < Q;
        const uint32_t tap = (q * m_cpt) >> 8, khi = tap / 3, kwi = tap - khi * 3;
        const uint32_t off = real ? (khi * PW + kwi) * g.ppitch + (q - tap * cpt) * 16 : 0u;
        v4i ah[MI], al[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const uint32_t r = (i * 16 + (lane & 15)) * g.apitch + q * 16;
            ah[i] = *reinterpret_cast<const v4i*>(a_hi + r);
            al[i] = *reinterpret_cast<const v4i*>(a_lo + r);
            rh[i] = bsum16(ah[i], rh[i]);
            rl[i] = bsum16(al[i], rl[i]);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            v4i bh = *reinterpret_cast<const v4i*>(p_hi + bbase[j] + off);
            v4i bl = *reinterpret_cast<const v4i*>(p_lo + bbase[j] + off);
            const int zl = (int)0x80808080u;
            bh = real ? bh : v4i{0, 0, 0, 0};
            bl = real ? bl : v4i{zl, zl, zl, zl};
            ch[j] = bsum16(bh, ch[j]);
            cl[j] = bsum16(bl, cl[j]);
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                hh[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bh, hh[i][j], 0, 0, 0);
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bl, mid[i][j], 0, 0, 0);
                ll[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bl, ll[i][j], 0, 0, 0);
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bh, mid[i][j], 0, 0, 0);
            }
        }
    }
    // totals over the four k chunks of a step (lanes l, l^16, l^32, l^48), as
    // sums of values: 256 * high + low + 128 per k position
    const uint32_t kp128 = 128u * 64u * g.nk;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint32_t cs = 256u * (uint32_t)ch[j] + (uint32_t)cl[j];
        cs += (uint32_t)__shfl_xor((int)cs, 16, 64);
        cs += (uint32_t)__shfl_xor((int)cs, 32, 64);
        if (lane < 16) colsum[(wave * 2 + j) * 16 + lane] = cs + kp128;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        uint32_t rs = 256u * (uint32_t)rh[i] + (uint32_t)rl[i];
        rs += (uint32_t)__shfl_xor((int)rs, 16, 64);
        rs += (uint32_t)__shfl_xor((int)rs, 32, 64);
        if (wave == 0 && lane < 16) rowsum[i * 16 + lane] = rs + kp128;
    }
    __syncthreads();   // every plane read is done: the tile may overwrite them

#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t v = ((uint32_t)hh[i][j][e] << 16) + ((uint32_t)mid[i][j][e] << 8) +
                                   (uint32_t)ll[i][j][e];
                tile[(i * 16 + (lane >> 4) * 4 + e) * kTilePitch + (wave * 2 + j) * 16 + (lane & 15)] = v;
            }
    __syncthreads();

    // Row-major finish: thread t covers 8 columns (half of tile row (t&15)/2)
    // of channels t>>4, +16, ...: sum corrections, bias, saturation, the fused
    // Add and activation, then the stores.
    const uint32_t chunk = tid & 15, ty = chunk >> 1, tx0 = (chunk & 1) * 8;
    const uint32_t oh = oh0 + ty, ow = ow0 + tx0;
    if (oh >= g.OH || ow >= g.OW) return;
    const uint32_t ncol = g.OW - ow < 8u ? g.OW - ow : 8u;
    const uint32_t kp_term = 16384u * 64u * g.nk;
    uint32_t cterm[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) cterm[q] = 128u * colsum[chunk * 8 + q] - kp_term;
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    const uint64_t obase = (uint64_t)n * g.y_img + (uint64_t)oh * g.OW + ow;
    const uint64_t mstride = (uint64_t)g.OH * g.OW;
    for (uint32_t m = tid >> 4; m < g.M; m += kThreads / 16) {
        const uint64_t o = obase + (uint64_t)m * mstride;
        int32_t add[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (g.epi.add_mode == 1u) {
            const int16_t* ap = g.epi.add + o;
            if (ncol == 8u && g.vw == 8u) {
                const v8s a = *reinterpret_cast<const v8s*>(ap);
#pragma unroll
                for (int q = 0; q < 8; ++q) add[q] = a[q];
            } else {
#pragma unroll
                for (int q = 0; q < 8; ++q) add[q] = (uint32_t)q < ncol ? ap[q] : 0;
            }
        }
        const uint32_t rs = 128u * rowsum[m] + (HAS_BIAS ? biasv[m] : 0u);
        int32_t yv[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t v = tile[m * kTilePitch + chunk * 8 + q] + cterm[q] + rs;
            yv[q] = q88::clamp(q88::add(q88::acc_to_data(v), add[q]), lo, hi);
        }
        int16_t* yp = g.y + o;
        if (ncol == 8u && g.vw == 8u) {
            v8s t;
#pragma unroll
            for (int q = 0; q < 8; ++q) t[q] = (short)yv[q];
            *reinterpret_cast<v8s*>(yp) = t;
        } else if (g.vw >= 4u) {   // ncol is 4 or 8
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if ((uint32_t)h * 4u < ncol) {
                    v4s t;
#pragma unroll
                    for (int q = 0; q < 4; ++q) t[q] = (short)yv[h * 4 + q];
                    *reinterpret_cast<v4s*>(yp + h * 4) = t;
                }
            }
        } else if (g.vw == 2u) {   // ncol is even
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                if ((uint32_t)h * 2u < ncol) {
                    v2s t;
                    t[0] = (short)yv[h * 2];
                    t[1] = (short)yv[h * 2 + 1];
                    *reinterpret_cast<v2s*>(yp + h * 2) = t;
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if ((uint32_t)q < ncol) yp[q] = (int16_t)yv[q];
        }
    }
}

inline bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

template <int MT, int S>
int launch_patch(const PatchArgs& g, uint32_t tiles, uint32_t lds, bool bias, hipStream_t s) {
    const void* k = bias ? (const void*)conv_patch<MT, S, true> : (const void*)conv_patch<MT, S, false>;
    if (lds > 65536u &&
        hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();
        return 1;   // not applicable: the caller takes the gather path
    }
    if (bias) hipLaunchKernelGGL((conv_patch<MT, S, true>), dim3(tiles), dim3(kThreads), lds, s, g);
    else hipLaunchKernelGGL((conv_patch<MT, S, false>), dim3(tiles), dim3(kThreads), lds, s, g);
    return cm_check_launch("conv_patch");
}

}  // namespace

// Returns 1 (nothing launched) when the shape is not one this kernel takes.
int cm_conv_patch_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                         uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                         uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                         uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                         uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc) {
    const hipStream_t s = lc.s;
    const EpiArgs ea = cm_epi_args(epi);
    if (kh != 3 || kw != 3 || dh != 1 || dw != 1 || sh != sw || (sh != 1 && sh != 2)) return 1;
    if (in_ch == 0 || in_ch > 64 || out_ch == 0 || out_ch > 64 || (in_ch * 9) % 8 != 0) return 1;
    if (!aligned(w, 16) || ea.add_mode > 1u) return 1;
    const uint64_t x_img = (uint64_t)in_ch * in_h * in_w;
    if (2 * x_img >= 0x80000000ull || (uint64_t)out_ch * 9 * in_ch * 2 >= 0x80000000ull) return 1;
    if (pad_top > 2 || pad_left > 2 || in_h >= (1u << 20) || in_w >= (1u << 20)) return 1;
    const uint32_t tiles_w = (out_w + TW - 1) / TW, tiles_h = (out_h + TH - 1) / TH;
    const uint64_t tiles = (uint64_t)tiles_w * tiles_h * batch;
    // Fewer tiles than a quarter of the CUs leave the chip idle: the gather
    // path splits K across blocks instead (measured slower here below 64).
    if (tiles < 64 || tiles > 0x7FFFFFFFull) return 1;

    PatchArgs g{};
    g.x = x; g.w = w; g.bias = bias; g.y = y;
    g.C = in_ch; g.H = in_h; g.W = in_w; g.M = out_ch; g.OH = out_h; g.OW = out_w;
    g.pt = pad_top; g.pl = pad_left;
    g.C16 = (in_ch + 15) / 16 * 16;
    g.nk = (9 * g.C16 + 63) / 64;
    g.apitch = g.nk * 64 + 16;                          // odd multiple of 16 bytes
    g.ppitch = (g.C16 / 16) % 2 ? g.C16 : g.C16 + 16;   // odd multiple of 16 bytes
    const uint32_t mt = out_ch <= 16 ? 16 : out_ch <= 32 ? 32 : 64;
    const uint32_t npos = sh == 1 ? PatchGeom<1>::NPOS : PatchGeom<2>::NPOS;
    g.p_off = 2 * mt * g.apitch;
    uint32_t lds = g.p_off + 2 * npos * g.ppitch;
    const uint32_t tile_bytes = mt * kTilePitch * 4;
    if (lds < tile_bytes) lds = tile_bytes;
    if (lds > 160u * 1024u - 2048u) return 1;
    if (lc.need) return CM_OK;   // dry run: this path uses no workspace
    g.tiles_w = tiles_w; g.tiles_h = tiles_h;
    g.div_tw = make_fastdiv(tiles_w);
    g.div_th = make_fastdiv(tiles_h);
    g.div_k = make_fastdiv(in_ch * 9);
    g.x_img_bytes = (uint32_t)(2 * x_img);
    g.x_img = x_img;
    g.y_img = (uint64_t)out_ch * out_h * out_w;
    g.epi = ea;
    // widest output access that keeps every row piece aligned and in one row
    g.vw = 8;
    while (g.vw > 1u) {
        const uint32_t v = g.vw;
        if (out_w % v == 0 && aligned(y, 2u * v) && (ea.add_mode != 1u || aligned(ea.add, 2u * v))) break;
        g.vw = v / 2u;
    }
    const bool b = bias != nullptr;
    const uint32_t t = (uint32_t)tiles;
    if (sh == 1) {
        if (mt == 16) return launch_patch<16, 1>(g, t, lds, b, s);
        if (mt == 32) return launch_patch<32, 1>(g, t, lds, b, s);
        return launch_patch<64, 1>(g, t, lds, b, s);
    }
    if (mt == 16) return launch_patch<16, 2>(g, t, lds, b, s);
    if (mt == 32) return launch_patch<32, 2>(g, t, lds, b, s);
    return launch_patch<64, 2>(g, t, lds, b, s);
}
