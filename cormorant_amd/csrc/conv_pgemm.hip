// conv_pgemm.hip -- standard convolution on int8 MFMA with the im2col operand
// read from an input patch in LDS and the weights pre-split into limb planes.
//
// Reference arithmetic (kernels/conv/kernel/ConvKernel.cpp:160-169, 171-249, 333):
//     acc = wrap32([bias << 8] + sum_{c,kh,kw valid} x * w),   y = sat16(acc >> 8).
//
// Two launches:
//   conv_wpack  splits the weights once per call into int8 limb planes in the
//               caller's workspace, in the k order the main kernel consumes, and
//               sums each output channel's weights (the limb identity's row sums);
//   conv_pgemm  one block per (128 output channels, 128 consecutive output
//               pixels of one image).  The input rows those pixels' windows touch
//               are loaded once per chunk of 64 channels and stored in LDS
//               channel-minor as limb planes, so the 16 k values one MFMA lane
//               supplies (16 channels of one tap at one pixel) are one 16-byte
//               LDS read: the B operand needs no per-step staging and no gather.
//               The per-step A tile is two 16-byte loads per thread from the
//               packed planes (L2-resident) straight into LDS.  No limb split,
//               transposition or load-address arithmetic runs in the k loop.
//
// Limbs and the exact sum are the GEMM kernel's: v = 256*vh + vl + 128 with
// vh = v >> 8, vl = (v & 255) - 128 (both int8), and
//     sum a*b = 65536*S_hh + 256*S_mid + S_ll + 128*(sum a + sum b) - 16384*Kp
// over Kp = 64 * steps k positions; a position holding a zero operand (padding
// channels, window taps outside the image, k past the chunk's taps) adds 0 to
// both sides.  Every term is taken modulo 2^32, the accumulator's wrap.
//
// Reduction order: chunk of 64 channels (c0 = 64*chunk), then q = tap*cpt + cg
// (cpt = 16-channel groups in the chunk, tap = kh_i*KW + kw_i), then 16
// channels; a k step is 4 consecutive q.
//
// Window geometry: with g = gcd(stride, dilation), every input row / column a
// tile touches is ih_first + g*r / g*col - pad_left, so the patch stores only
// those: row r, column col hold x[c][ih_first + g*r][g*col - pad_left]; pixel
// (oh, ow) at tap (kh_i, kw_i) reads row (oh - oh_first)*S' + kh_i*D', column
// ow*S' + kw_i*D' (S' = stride/g, D' = dilation/g).
#include "cm_internal.h"
#include "q88.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr uint32_t kPackTile = 2u * BM * 64u; // packed bytes per (row tile, step): hi then lo
constexpr int kMaxQ = 256;                    // q table entries (taps * 4 <= 256)

struct PgArgs {
    const int16_t* x;
    const uint8_t* wpk;          // packed weight limb planes
    const uint32_t* wsum;        // [M] sum of each output channel's weights (wrapping)
    const int16_t* bias;
    int16_t* y;
    uint32_t C, H, W, M, OH, OW, P;   // P = OH * OW
    uint32_t KW, taps, S, Sg, Dg, g, pt, pl;
    uint32_t nchunks, steps;     // channel chunks; k steps over all chunks
    uint32_t PW, ppitch;         // patch positions per row; LDS bytes per position
    uint32_t prows, npos;        // patch rows / positions staged per block (the most any block needs)
    uint32_t p_plane;            // LDS bytes of one patch limb plane (the zero slot included)
    uint32_t zslot;              // byte offset in each plane of 16 bytes holding the limbs of 0
    uint32_t lhc, wr, nh;        // padding columns: left [0, lhc), right [wr, wr + nh - lhc)
    uint32_t cpt_last;           // 16-channel groups of the last chunk
    uint32_t R, bands;           // output rows per block; bands per image
    FastDiv div_bands, div_ow, div_npos, div_pw, div_nv, div_prows, div_nh, div_kw, div_cpt4, div_cpt_last;
    uint32_t vw;                 // output / Add access width in elements (8 or 1)
    uint32_t x_img_bytes, pk_bytes;
    uint64_t x_img, y_img;
    EpiArgs epi;
};

__device__ __forceinline__ int32_t bsum16(v4i v, int32_t acc) {
#pragma unroll
    for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_sdot4(v[q], 0x01010101, acc, false);
    return acc;
}
__device__ __forceinline__ uint32_t hi_byte(int32_t v) { return (uint32_t)(v >> 8) & 0xFFu; }
__device__ __forceinline__ uint32_t lo_byte(int32_t v) { return ((uint32_t)v & 0xFFu) ^ 0x80u; }
__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// ------------------------------------------------------------ weight pack --
// One block per output channel row m of a 128-row tile (rows past M are packed
// as zeros).  Word w of a (row tile, step) plane row covers k bytes 4w..4w+3 of
// the step: sub-chunk q = 4*step_in_chunk + w/4, channels 16*(q % cpt) + 4*(w%4)
// + 0..3 of the chunk, tap q / cpt.
struct PackArgs {
    const int16_t* w;
    uint8_t* wpk;
    uint32_t* wsum;
    uint32_t C, M, taps, nchunks, steps, steps_full;   // steps_full = taps (a full chunk)
};

__global__ __launch_bounds__(256) void conv_wpack(PackArgs a) {
    const uint32_t m = blockIdx.x;   // 0 .. Mpad-1
    const uint32_t mt = m / BM, r = m % BM;
    const bool mok = m < a.M;
    const int16_t* wrow = a.w + (uint64_t)(mok ? m : 0u) * a.C * a.taps;
    uint32_t sum = 0;
    const uint32_t words = a.steps * 16u;
    for (uint32_t i = threadIdx.x; i < words; i += 256) {
        const uint32_t gs = i >> 4, wd = i & 15u;
        const uint32_t ch = min(gs / a.steps_full, a.nchunks - 1u);
        const uint32_t ls = gs - ch * a.steps_full;
        const uint32_t c0 = ch * 64u;
        const uint32_t cc = min(64u, a.C - c0);
        const uint32_t cpt = (cc + 15u) / 16u;
        const uint32_t q = ls * 4u + (wd >> 2);
        const uint32_t tap = q / cpt, cg = q - tap * cpt;
        uint32_t hw = 0, lw = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t cl = cg * 16u + (wd & 3u) * 4u + j;
            const bool ok = mok && tap < a.taps && cl < cc;
            const int32_t v = ok ? (int32_t)wrow[(uint64_t)(c0 + cl) * a.taps + tap] : 0;
            sum += (uint32_t)v;
            hw |= hi_byte(v) << (8 * j);
            lw |= lo_byte(v) << (8 * j);
        }
        uint8_t* dst = a.wpk + (uint64_t)(mt * a.steps + gs) * kPackTile + r * 64u + wd * 4u;
        *reinterpret_cast<uint32_t*>(dst) = hw;
        *reinterpret_cast<uint32_t*>(dst + BM * 64u) = lw;
    }
    // row sum (every real weight once; padding adds 0)
    __shared__ uint32_t red[256];
    red[threadIdx.x] = sum;
    __syncthreads();
    for (uint32_t s = 128; s > 0; s >>= 1) {
        if (threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0 && mok) a.wsum[m] = red[0];
}

// ------------------------------------------------------------- main kernel --
// Block: 256 threads = 4 waves (2 x 2), 128 output channels of one band of R
// output rows of one image, computed in sub-tiles of 64 pixels (flattened over
// the band); wave tile 64 channels x 32 pixels (4 x 2 MFMA 16x16x64 tiles,
// three accumulator sets).  With one channel chunk the band's input rows are
// staged into the LDS patch once and every sub-tile reads them; with more
// chunks each sub-tile restages every chunk.  Each wave loads its A fragments
// straight from the packed planes (a row tile of one limb is 16 rows x 64
// bytes, 1 KB contiguous: one 16-byte load per lane), one step ahead, so the k
// loop has no barrier and no LDS writes.  A sub-tile's results go out through
// a 64-row LDS tile in two halves, as 16-byte stores of 8 neighbouring pixels.
constexpr int kPgThreads = 256;
constexpr int PBN = 64;          // pixels per sub-tile
constexpr int kTilePitch = 68;   // epilogue half tile: words per row (64 + 4)

// VEC: patch rows loaded 16 bytes at a time with g = VEC; 0 = per element.
// MULTI: more than one channel chunk (restaged inside the k loop, with fewer
// loads in flight while the accumulators are live).
template <bool HAS_BIAS, int VEC, bool MULTI>
__global__ __launch_bounds__(kPgThreads, 2) void conv_pgemm(PgArgs g) {
    constexpr int kPB = MULTI ? 1 : 3;   // 16-byte staging tasks per thread in flight
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t colterm_s[PBN];                // 128 * column sum - 16384 * Kp
    __shared__ __align__(16) uint32_t rowterm_s[BM];   // 128 * row sum + bias << 8
    __shared__ int32_t qtab[kMaxQ];   // per sub-chunk q: patch byte offset of its tap and group
    uint8_t* p_hi = lds;
    uint8_t* p_lo = lds + g.p_plane;
    uint32_t* tile = reinterpret_cast<uint32_t*>(lds + 2 * g.p_plane);   // [64][kTilePitch]

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wrow = (wave >> 1) * 64, wcol = (wave & 1) * 32;
    const uint32_t mt = blockIdx.y, row0 = mt * BM;
    const uint32_t n = fdiv(blockIdx.x, g.div_bands);
    const uint32_t oh0 = (blockIdx.x - n * g.bands) * g.R;
    const uint32_t bp0 = oh0 * g.OW;                              // the band's first pixel
    const uint32_t bp1 = min(oh0 + g.R, g.OH) * g.OW;             // one past its last
    const int32_t ih_first = (int32_t)(oh0 * g.S) - (int32_t)g.pt;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(g.x + (uint64_t)n * g.x_img, g.x_img_bytes);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(reinterpret_cast<const int16_t*>(g.wpk), g.pk_bytes);
    const uint32_t hw_in = g.H * g.W;

    if (tid < BM) {
        const uint32_t m = row0 + tid;
        const uint32_t b = HAS_BIAS && m < g.M ? (uint32_t)((int32_t)g.bias[m] * 256) : 0u;
        rowterm_s[tid] = (m < g.M ? 128u * g.wsum[m] : 0u) + b;
    }
    if (tid == 0) {   // the zero slot: 16 bytes of each plane holding the limbs of 0
        *reinterpret_cast<v4u*>(p_hi + g.zslot) = v4u{0u, 0u, 0u, 0u};
        *reinterpret_cast<v4u*>(p_lo + g.zslot) = v4u{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
    }

    // A fragments of step gs: row tile i of the wave's 64 rows, hi and lo planes
    // (steps past the last one read another row tile's data or, past the buffer,
    // 0; neither is used)
    const uint32_t a_src = (mt * g.steps) * kPackTile + (wrow + (lane & 15)) * 64u + (lane >> 4) * 16u;
    auto a_load = [&](uint32_t gs, v4i (&ah)[4], v4i (&al)[4]) {
        const uint32_t off = a_src + gs * kPackTile;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ah[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wrs, off + i * 1024u, 0, 0));
            al[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                wrs, off + BM * 64u + i * 1024u, 0, 0));
        }
    };

    // Patch staging of one chunk (the band's rows).  Rows outside the image and
    // channels past C read 0 through the buffer range.
    auto stage_patch = [&](uint32_t c0, uint32_t cpt, const FastDiv& div_cpt) {
        const uint32_t ncq = cpt * 4u;
        if constexpr (VEC == 0) {
            // per element: task e = (channel quad cq, position), position fastest
            constexpr int kPE = 4;
            const uint32_t ntask = ncq * g.npos;
            for (uint32_t b0 = 0; b0 < ntask; b0 += kPgThreads * kPE) {
                uint32_t v[kPE][4];
                uint32_t dst[kPE];
#pragma unroll
                for (int u = 0; u < kPE; ++u) {
                    const uint32_t e = b0 + u * kPgThreads + tid;
                    const uint32_t cq = fdiv(e, g.div_npos), pos = e - cq * g.npos;
                    const uint32_t r = fdiv(pos, g.div_pw), col = pos - r * g.PW;
                    const int32_t ih = ih_first + (int32_t)(r * g.g);
                    const int32_t iw = (int32_t)(col * g.g) - (int32_t)g.pl;
                    const uint32_t okp = (uint32_t)(e < ntask) & (uint32_t)((uint32_t)ih < g.H) &
                                         (uint32_t)((uint32_t)iw < g.W);
                    const uint32_t c = c0 + cq * 4u;
                    const uint32_t base = (c * hw_in + (uint32_t)ih * g.W + (uint32_t)iw) * 2u;
                    dst[u] = e < ntask ? pos * g.ppitch + cq * 4u : 0xFFFFFFFFu;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const uint32_t ok = okp & (uint32_t)(c + jj < g.C);
                        const uint32_t off = ((base + jj * hw_in * 2u) & 0x7FFFFFFFu) | ((ok ^ 1u) << 31);
                        v[u][jj] = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(xrs, off, 0, 0);
                    }
                }
#pragma unroll
                for (int u = 0; u < kPE; ++u) {
                    if (dst[u] == 0xFFFFFFFFu) continue;
                    uint32_t wh = 0, wl = 0;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int32_t xv = (int32_t)(int16_t)v[u][jj];
                        wh |= hi_byte(xv) << (8 * jj);
                        wl |= lo_byte(xv) << (8 * jj);
                    }
                    *reinterpret_cast<uint32_t*>(p_hi + dst[u]) = wh;
                    *reinterpret_cast<uint32_t*>(p_lo + dst[u]) = wl;
                }
            }
        } else {
            // 16 bytes at a time: task e = (channel quad cq, patch row r, 8-column
            // group v of the input row); four loads (one per channel) give 8 input
            // columns, of which every VEC-th lands in the patch: position
            // col = (iw + pl) / VEC for iw = pl (mod VEC).  Input rows are 16-byte
            // aligned (W % 8 == 0), and patch rows are wide enough for all of
            // them (PW >= lh + W / VEC), so no write needs a condition.
            const uint32_t nv = g.W / 8u;
            const uint32_t ntask = ncq * g.prows * nv;
            const uint32_t lh = (g.pl + VEC - 1u) / VEC;   // patch column of the first input column used
            for (uint32_t b0 = 0; b0 < ntask; b0 += kPgThreads * kPB) {
                v4u d[kPB][4];
                uint32_t dst0[kPB];
#pragma unroll
                for (int u = 0; u < kPB; ++u) {
                    const uint32_t e = b0 + u * kPgThreads + tid;
                    const uint32_t cqr = fdiv(e, g.div_nv), vv = e - cqr * nv;
                    const uint32_t cq = fdiv(cqr, g.div_prows), r = cqr - cq * g.prows;
                    const int32_t ih = ih_first + (int32_t)(r * VEC);
                    const uint32_t okr = (uint32_t)(e < ntask) & (uint32_t)((uint32_t)ih < g.H);
                    const uint32_t c = c0 + cq * 4u;
                    const uint32_t base = (c * hw_in + (uint32_t)ih * g.W + vv * 8u) * 2u;
                    dst0[u] = e < ntask ? (r * g.PW + vv * (8u / VEC) + lh) * g.ppitch + cq * 4u
                                        : 0xFFFFFFFFu;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const uint32_t ok = okr & (uint32_t)(c + jj < g.C);
                        const uint32_t off = ((base + jj * hw_in * 2u) & 0x7FFFFFFFu) | ((ok ^ 1u) << 31);
                        d[u][jj] = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
                    }
                }
#pragma unroll
                for (int u = 0; u < kPB; ++u) {
                    if (dst0[u] == 0xFFFFFFFFu) continue;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {   // dword k holds input columns 8v+2k, 8v+2k+1
                        const uint32_t d0 = d[u][0][k], d1 = d[u][1][k], d2 = d[u][2][k], d3 = d[u][3][k];
                        const uint32_t t01 = __builtin_amdgcn_perm(d1, d0, 0x07030501u);
                        const uint32_t t23 = __builtin_amdgcn_perm(d3, d2, 0x07030501u);
                        const uint32_t u01 = __builtin_amdgcn_perm(d1, d0, 0x06020400u);
                        const uint32_t u23 = __builtin_amdgcn_perm(d3, d2, 0x06020400u);
#pragma unroll
                        for (int h = 0; h < 2; ++h) {   // input column 8v + 2k + h
                            if (VEC == 2 && (uint32_t)h != (g.pl & 1u)) continue;
                            const uint32_t sel = h ? 0x07060302u : 0x05040100u;
                            const uint32_t dst = dst0[u] + (VEC == 1 ? 2u * k + h : (uint32_t)k) * g.ppitch;
                            *reinterpret_cast<uint32_t*>(p_hi + dst) = __builtin_amdgcn_perm(t23, t01, sel);
                            *reinterpret_cast<uint32_t*>(p_lo + dst) =
                                __builtin_amdgcn_perm(u23, u01, sel) ^ 0x80808080u;
                        }
                    }
                }
            }
            // padding columns (input columns outside the row) that a window reads:
            // left [0, lhc), right [wr, PWr)
            const uint32_t nhalo = ncq * g.prows * g.nh;
            for (uint32_t e = tid; e < nhalo; e += kPgThreads) {
                const uint32_t cqr = fdiv(e, g.div_nh), hcol = e - cqr * g.nh;
                const uint32_t cq = fdiv(cqr, g.div_prows), r = cqr - cq * g.prows;
                const uint32_t col = hcol < g.lhc ? hcol : g.wr + (hcol - g.lhc);
                const uint32_t dst = (r * g.PW + col) * g.ppitch + cq * 4u;
                *reinterpret_cast<uint32_t*>(p_hi + dst) = 0u;
                *reinterpret_cast<uint32_t*>(p_lo + dst) = 0x80808080u;
            }
        }
        // q table of the chunk: q = tap * cpt + cg -> byte offset of (tap, group)
        // from a pixel's window origin; -1 past the chunk's last sub-chunk
        for (uint32_t q = tid; q < (uint32_t)kMaxQ; q += kPgThreads) {
            const uint32_t tap = fdiv(q, div_cpt), cg = q - tap * cpt;
            const uint32_t khi = fdiv(tap, g.div_kw), kwi = tap - khi * g.KW;
            qtab[q] = tap < g.taps ? (int32_t)(((khi * g.PW + kwi) * g.Dg) * g.ppitch + cg * 16u) : -1;
        }
    };

    const bool sums = (wave >> 1) == 0;   // one wave row publishes the column sums
    const uint32_t kp128 = 128u * 64u * g.steps;
    const uint32_t kp_term = 16384u * 64u * g.steps;
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    const uint32_t nsub = (bp1 - bp0 + PBN - 1) / PBN;
    v4i fa_h[2][4], fa_l[2][4];
    uint32_t gs = 0;   // global k step of the next MFMA step, over all sub-tiles

    for (uint32_t sub = 0; sub < nsub; ++sub) {
        const uint32_t p0 = bp0 + sub * PBN;
        // the first chunk's patch (with one chunk: staged once for every sub-tile),
        // before the accumulators and A fragments of this sub-tile are live
        if (sub == 0 || MULTI) {
            if (sub) __syncthreads();   // every wave is done with the previous patch
            stage_patch(0u, MULTI ? 4u : g.cpt_last, MULTI ? g.div_cpt4 : g.div_cpt_last);
            __syncthreads();
        }
        if (sub == 0) a_load(0, fa_h[0], fa_l[0]);
        // byte offset in the patch of the window origin of this lane's pixel in
        // each column tile: row (oh - oh0) * S', column ow * S'
        uint32_t pbase[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t px = min(p0 + wcol + j * 16 + (lane & 15), bp1 - 1u);   // past the band: any of its pixels
            const uint32_t oh = fdiv(px, g.div_ow), ow = px - oh * g.OW;
            pbase[j] = (((oh - oh0) * g.PW + ow) * g.Sg) * g.ppitch;
        }
        v4i hh[4][2], mid[4][2], ll[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                hh[i][j] = v4i{0, 0, 0, 0}; mid[i][j] = v4i{0, 0, 0, 0}; ll[i][j] = v4i{0, 0, 0, 0};
            }
        int32_t csh[2] = {0, 0}, csl[2] = {0, 0};

        auto mfma_step = [&](uint32_t ls, const v4i (&ah)[4], const v4i (&al)[4]) {
            const int32_t qo = qtab[ls * 4u + (lane >> 4)];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                // past the chunk's last sub-chunk: the zero slot (the limbs of 0)
                const uint32_t a = qo >= 0 ? pbase[j] + (uint32_t)qo : g.zslot;
                const v4i bh = *reinterpret_cast<const v4i*>(p_hi + a);
                const v4i bl = *reinterpret_cast<const v4i*>(p_lo + a);
                if (sums) {
                    csh[j] = bsum16(bh, csh[j]);
                    csl[j] = bsum16(bl, csl[j]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    hh[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bh, hh[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bl, mid[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ll[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bl, ll[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bh, mid[i][j], 0, 0, 0);
            }
        };

        // k loop over the chunks (steps gs of the packed planes restart at 0 for
        // each sub-tile: the A fragments of the next step load while this step's
        // MFMAs run; the pairs keep the register sets fixed at compile time)
        uint32_t ks = 0;   // k step within this sub-tile
        for (uint32_t ch = 0; ch < (MULTI ? g.nchunks : 1u); ++ch) {
            const uint32_t c0 = ch * 64u;
            const bool last = ch + 1 == g.nchunks;
            const uint32_t cpt = last ? g.cpt_last : 4u;
            const uint32_t nst = (g.taps * cpt + 3u) / 4u;
            if (MULTI && ch) {   // later chunks: restaged here
                __syncthreads();   // every wave is done with the previous chunk's patch
                stage_patch(c0, cpt, last ? g.div_cpt_last : g.div_cpt4);
                __syncthreads();
            }
            uint32_t ls = 0;
            if (gs & 1u) {
                a_load(ks + 1 < g.steps ? ks + 1 : 0u, fa_h[0], fa_l[0]);
                mfma_step(ls, fa_h[1], fa_l[1]);
                ++ls; ++gs; ++ks;
            }
            for (; ls + 2 <= nst; ls += 2, gs += 2, ks += 2) {
                a_load(ks + 1 < g.steps ? ks + 1 : 0u, fa_h[1], fa_l[1]);
                mfma_step(ls, fa_h[0], fa_l[0]);
                a_load(ks + 2 < g.steps ? ks + 2 : ks + 2 - g.steps, fa_h[0], fa_l[0]);
                mfma_step(ls + 1, fa_h[1], fa_l[1]);
            }
            if (ls < nst) {
                a_load(ks + 1 < g.steps ? ks + 1 : 0u, fa_h[1], fa_l[1]);
                mfma_step(ls, fa_h[0], fa_l[0]);
                ++gs; ++ks;
            }
        }

        // column terms of this sub-tile (sums of values over the four lane
        // groups: 256 * high + low + 128 per k position); the barrier keeps the
        // previous sub-tile's epilogue reads ahead of these writes
        __syncthreads();
        if (sums) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t cs = 256u * (uint32_t)csh[j] + (uint32_t)csl[j];
                cs += (uint32_t)__shfl_xor((int)cs, 16, 64);
                cs += (uint32_t)__shfl_xor((int)cs, 32, 64);
                if (lane < 16) colterm_s[wcol + j * 16 + lane] = 128u * (cs + kp128) - kp_term;
            }
        }

        // epilogue: two halves of 64 output channels through the LDS tile; thread t
        // then finishes pixels [c8, c8 + 8) of channels rb and rb + 32 of the half
        const uint32_t c8 = (tid & 7) * 8, rb = tid >> 3;
        const uint32_t px0 = p0 + c8;
        const uint32_t ncol = px0 < bp1 ? (bp1 - px0 < 8u ? bp1 - px0 : 8u) : 0u;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            __syncthreads();   // column terms published; the tile is free again
            if ((wave >> 1) == (uint32_t)half) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const uint32_t v = ((uint32_t)hh[i][j][e] << 16) +
                                               ((uint32_t)mid[i][j][e] << 8) + (uint32_t)ll[i][j][e];
                            tile[(i * 16 + (lane >> 4) * 4 + e) * kTilePitch + wcol + j * 16 + (lane & 15)] = v;
                        }
            }
            __syncthreads();
            if (ncol) {
                uint32_t cterm[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) cterm[q] = colterm_s[c8 + q];
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    const uint32_t r = rb + rr * 32;             // row within the half
                    const uint32_t m = row0 + half * 64 + r;
                    if (m >= g.M) continue;
                    const uint64_t o = (uint64_t)n * g.y_img + (uint64_t)m * g.P + px0;
                    int32_t add[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                    if (g.epi.add_mode == 1u) {
                        const int16_t* ap = g.epi.add + o;
                        if (ncol == 8u && g.vw == 8u) {
                            const v4u a = *reinterpret_cast<const v4u*>(ap);
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                add[2 * q] = (int32_t)(int16_t)(a[q] & 0xFFFFu);
                                add[2 * q + 1] = (int32_t)a[q] >> 16;
                            }
                        } else {
#pragma unroll
                            for (int q = 0; q < 8; ++q) add[q] = (uint32_t)q < ncol ? ap[q] : 0;
                        }
                    }
                    const uint32_t rs = rowterm_s[half * 64 + r];
                    const v4u t0 = *reinterpret_cast<const v4u*>(&tile[r * kTilePitch + c8]);
                    const v4u t1 = *reinterpret_cast<const v4u*>(&tile[r * kTilePitch + c8 + 4]);
                    int32_t yv[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const uint32_t v = (q < 4 ? t0[q] : t1[q - 4]) + cterm[q] + rs;
                        yv[q] = q88::clamp(q88::add(q88::acc_to_data(v), add[q]), lo, hi);
                    }
                    int16_t* yp = g.y + o;
                    if (ncol == 8u && g.vw == 8u) {
                        *reinterpret_cast<v4u*>(yp) = v4u{pack2(yv[0], yv[1]), pack2(yv[2], yv[3]),
                                                          pack2(yv[4], yv[5]), pack2(yv[6], yv[7])};
                    } else {
#pragma unroll
                        for (int q = 0; q < 8; ++q)
                            if ((uint32_t)q < ncol) yp[q] = (int16_t)yv[q];
                    }
                }
            }
        }
    }
}

inline bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

uint32_t gcd(uint32_t a, uint32_t b) {
    while (b) { const uint32_t t = a % b; a = b; b = t; }
    return a;
}

}  // namespace

// Returns 1 (launching nothing) when the shape does not suit this path or the
// workspace is too small; with lc.need set, records the workspace it needs.
int cm_conv_pgemm_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                         uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                         uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                         uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                         uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc) {
    const EpiArgs ea = cm_epi_args(epi);
    if (in_ch == 0 || out_ch == 0 || kh == 0 || kw == 0 || sh == 0 || dh == 0) return 1;
    // one stride / dilation pair for both axes keeps the patch rows and columns alike
    if (sh != sw || dh != dw || ea.add_mode > 1u) return 1;
    const uint32_t taps = kh * kw;
    if (taps * 4u > (uint32_t)kMaxQ) return 1;
    const uint64_t P = (uint64_t)out_h * out_w;
    const uint64_t x_img = (uint64_t)in_ch * in_h * in_w;
    if (P == 0 || 2 * x_img >= 0x80000000ull || P >= (1u << 24) || in_h >= (1u << 20) ||
        in_w >= (1u << 20) || out_w > 4096 || pad_top >= in_h + kh * dh || pad_left >= in_w + kw * dw)
        return 1;
    const uint32_t mtiles = (out_ch + BM - 1) / BM;
    const uint32_t gg = gcd(sh, dh), Sg = sh / gg, Dg = dh / gg;
    if ((uint64_t)out_ch * P * 2 >= 0x80000000ull) return 1;
    // 16-byte patch loads: rows 16-byte aligned, and g = 1 or 2
    const uint32_t vec = (in_w % 8 == 0 && aligned(x, 16) && (gg == 1 || gg == 2)) ? gg : 0u;
    // patch columns a window reaches; with 16-byte loads the rows are widened to
    // hold every input column (PW >= lh + W / vec)
    const uint32_t PWr = (out_w - 1) * Sg + (kw - 1) * Dg + 1;
    const uint32_t lh = vec ? (pad_left + vec - 1) / vec : 0u;
    const uint32_t wr = vec ? lh + in_w / vec : 0u;
    const uint32_t PW = vec && wr > PWr ? wr : PWr;
    const uint32_t lhc = lh < PWr ? lh : PWr;
    const uint32_t nh = lhc + (PWr > wr ? PWr - wr : 0u);
    const uint32_t nchunks = (in_ch + 63) / 64;
    const uint32_t cpt_max = nchunks > 1 ? 4u : (in_ch + 15) / 16;
    const uint32_t ppitch = cpt_max % 2 ? cpt_max * 16 : cpt_max * 16 + 16;   // odd multiple of 16
    const uint64_t tile_bytes = 64ull * kTilePitch * 4;
    // Band of R output rows per block: the most rows (up to 8) that keep two
    // blocks per CU in LDS and the grid at >= 400 blocks (else >= 200); sub-tiles
    // of 64 pixels must be mostly full (>= 3/4 of the lanes over the whole band)
    uint32_t R = 0;
    uint64_t best_lds = 0;
    for (uint32_t min_blocks : {400u, 200u}) {
        for (uint32_t r = 1; r <= 8 && r <= out_h; ++r) {
            const uint64_t px = (uint64_t)r * out_w;
            const uint64_t bands = (out_h + r - 1) / r;
            const uint64_t blocks = bands * batch * mtiles;
            const uint64_t prows = (uint64_t)(r - 1) * Sg + (uint64_t)(kh - 1) * Dg + 1;
            const uint64_t lds = 2 * (prows * PW * ppitch + 16) + tile_bytes;
            const bool fill = px * 4 >= ((px + PBN - 1) / PBN) * PBN * 3;
            if (blocks < min_blocks || lds > 76u * 1024u || !fill) continue;
            R = r;
            best_lds = lds;
        }
        if (R) break;
    }
    if (R == 0) return 1;
    const uint32_t bands = (out_h + R - 1) / R;
    const uint64_t blocks = (uint64_t)bands * batch * mtiles;
    if (blocks > 0x7FFFFFFFull) return 1;
    const uint32_t prmax = (R - 1) * Sg + (kh - 1) * Dg + 1;
    const uint64_t zslot = (uint64_t)prmax * PW * ppitch;
    const uint64_t p_plane = zslot + 16;
    const uint64_t lds = best_lds;
    const uint32_t last_cpt = (in_ch - (nchunks - 1) * 64 + 15) / 16;
    const uint32_t steps = (nchunks - 1) * taps + (taps * last_cpt + 3) / 4;
    const uint64_t pk_bytes = (uint64_t)mtiles * steps * kPackTile;
    const uint64_t need = pk_bytes + 4ull * mtiles * BM;
    if (pk_bytes >= 0x80000000ull) return 1;
    if (lc.need) {
        if (need > *lc.need) *lc.need = need;
        return CM_OK;
    }
    if (!lc.ws || lc.ws_bytes < need || !aligned(lc.ws, 16)) return 1;

    uint8_t* wpk = static_cast<uint8_t*>(lc.ws);
    uint32_t* wsum = reinterpret_cast<uint32_t*>(wpk + pk_bytes);
    PackArgs pa{w, wpk, wsum, in_ch, out_ch, taps, nchunks, steps, taps};
    hipLaunchKernelGGL(conv_wpack, dim3(mtiles * BM), dim3(256), 0, lc.s, pa);
    int rc = cm_check_launch("conv_wpack");
    if (rc) return rc;

    PgArgs g{};
    g.x = x; g.wpk = wpk; g.wsum = wsum; g.bias = bias; g.y = y;
    g.C = in_ch; g.H = in_h; g.W = in_w; g.M = out_ch; g.OH = out_h; g.OW = out_w; g.P = (uint32_t)P;
    g.KW = kw; g.taps = taps; g.S = sh; g.Sg = Sg; g.Dg = Dg; g.g = gg; g.pt = pad_top; g.pl = pad_left;
    g.nchunks = nchunks; g.steps = steps;
    g.PW = PW; g.ppitch = ppitch; g.p_plane = (uint32_t)p_plane; g.zslot = (uint32_t)zslot;
    g.lhc = lhc; g.wr = wr; g.nh = nh;
    g.cpt_last = last_cpt;
    g.R = R; g.bands = bands;
    g.prows = prmax;
    g.npos = prmax * PW;
    g.div_bands = make_fastdiv(bands);
    g.div_ow = make_fastdiv(out_w);
    g.div_npos = make_fastdiv(g.npos);
    g.div_pw = make_fastdiv(PW);
    g.div_nv = make_fastdiv(in_w / 8 ? in_w / 8 : 1);
    g.div_prows = make_fastdiv(prmax);
    g.div_nh = make_fastdiv(nh ? nh : 1);
    g.div_kw = make_fastdiv(kw);
    g.div_cpt4 = make_fastdiv(4);
    g.div_cpt_last = make_fastdiv(last_cpt);
    g.x_img_bytes = (uint32_t)(2 * x_img);
    g.pk_bytes = (uint32_t)pk_bytes;
    g.x_img = x_img;
    g.y_img = (uint64_t)out_ch * P;
    g.epi = ea;
    // 16-byte output accesses: every run of 8 pixels starts 16-byte aligned
    // (bands start at multiples of R * OW pixels, sub-tiles at multiples of 64)
    g.vw = P % 8 == 0 && (uint64_t)R * out_w % 8 == 0 && aligned(y, 16) &&
                   (ea.add_mode != 1u || aligned(ea.add, 16))
               ? 8u
               : 1u;
    const void* k = nullptr;
#define CM_PG_PICK(B, M) (vec == 1 ? (const void*)conv_pgemm<B, 1, M> \
                          : vec == 2 ? (const void*)conv_pgemm<B, 2, M> : (const void*)conv_pgemm<B, 0, M>)
    if (nchunks > 1) k = bias ? CM_PG_PICK(true, true) : CM_PG_PICK(false, true);
    else k = bias ? CM_PG_PICK(true, false) : CM_PG_PICK(false, false);
#undef CM_PG_PICK
    if (lds > 65536u &&
        hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();
        return cm_set_error(CM_ERR_HIP, "conv_pgemm: %llu bytes of LDS refused", (unsigned long long)lds);
    }
    const dim3 grid((uint32_t)(bands * batch), mtiles);
    void* kargs[] = {&g};
    const hipError_t e = hipLaunchKernel(k, grid, dim3(kPgThreads), kargs, (size_t)lds, lc.s);
    if (e != hipSuccess) return cm_set_error(CM_ERR_HIP, "conv_pgemm: %s", hipGetErrorString(e));
    return cm_check_launch("conv_pgemm");
}
