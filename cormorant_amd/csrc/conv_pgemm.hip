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
//   conv_pgemm  one block per (128 output channels, range of L consecutive
//               output pixels of one image; L is chosen so the blocks spread
//               evenly over the CUs).  The input rows the range's windows touch
//               are loaded once (every channel, when they fit in LDS; else in
//               chunks of 64 channels) and stored in LDS channel-minor as limb
//               planes, so the 16 k values one MFMA lane
//               supplies (16 channels of one tap at one pixel) are one 16-byte
//               LDS read: the B operand needs no per-step staging and no gather.
//               Each wave's A fragments are 16-byte loads from the packed planes
//               (L2-resident).  No limb split, transposition, column sum or
//               load-address arithmetic beyond one add per tile runs in the k
//               loop.
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
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "cm_internal.h"
#include "q88.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr uint32_t kMaxTB = 128;   // output channels per row tile: 32, 64 or 128
constexpr int kMaxQ = 256;                    // q table entries (taps * 4 <= 256)

struct PgArgs {
    const int16_t* x;
    const uint8_t* wpk;          // packed weight limb planes
    const uint32_t* wsum;        // [M] sum of each output channel's weights (wrapping)
    const uint32_t* wfit;        // [M] 1 when every weight of the row is in [-128, 127]
    const int16_t* bias;
    int16_t* y;
    uint32_t C, H, W, M, OH, OW, P;   // P = OH * OW
    uint32_t KW, taps, S, Sg, Dg, g, pt, pl;
    uint32_t khspan;             // patch rows one output row's windows span: (KH - 1) * D' + 1
    uint32_t nchunks, steps;     // channel chunks; k steps over all chunks
    uint32_t PW, ppitch;         // patch positions per row; LDS bytes per position
    uint32_t prows, npos;        // patch rows / positions the LDS holds (the most any block needs)
    uint32_t p_plane;            // LDS bytes of one patch limb plane (the zero slot included)
    uint32_t zslot;              // byte offset in each plane of 16 bytes holding the limbs of 0
    uint32_t spos_off, epi_off;  // LDS byte offsets of the position sums and the epilogue tiles
    uint32_t lhc, wr, nh;        // padding columns: left [0, lhc), right [wr, wr + nh - lhc)
    uint32_t stage_g;            // 16-byte staging: (row, column group) pair groups per block
    uint32_t cpt_last;           // 16-channel groups of the last chunk
    uint32_t cpt_all;            // without MULTI: 16-channel groups the patch holds (every chunk)
    uint32_t nfull;              // without MULTI: full 64-channel chunks before the last one
    uint32_t L, rpi, rpi_n;      // output pixels per block; ranges per image; ranges per row tile
    FastDiv div_npr, div_nbm, div_rpi, div_ow, div_npos, div_pw, div_nv, div_prows, div_nh, div_kw, div_cpt4, div_cpt_last, div_t4;
    uint32_t vw;                 // output / Add access width in elements (8 or 1)
    uint32_t add_w4;             // Add runs 4-byte aligned (P even, operand 4-byte aligned)
    uint32_t x_img_bytes, pk_bytes;   // pk_bytes: both packed layouts (limb planes, then int8)
    uint32_t pk8_off;            // byte offset of the int8 plane
    uint64_t x_img, y_img;
    EpiArgs epi;
    // PAIR: a 1x1 convolution (M2 output channels) applied to this convolution's
    // output, which never leaves LDS; y, y_img and epi then describe the 1x1's
    // output, act1 the activation of the middle tensor
    const uint8_t* wpk2;         // the 1x1's packed weight planes (32-row tiles)
    const uint32_t* wsum2;       // [M2] its weight row sums
    const uint32_t* wfit2;       // [M2] 1 when the row's weights are all int8
    const int16_t* bias2;
    uint32_t M2, steps2, HP;     // 1x1 output channels; its k steps; LDS bytes per middle-tile pixel
    uint32_t hp_off, cs_off, rt2_off;   // LDS: middle-tile planes, pixel column sums, 1x1 row terms
    uint32_t pk2_bytes, pk2_8off;       // buffer range of the 1x1's planes; offset of its int8 plane
    uint32_t act1;
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
// One block per output channel row m of a row tile (rows past M are packed as
// zeros).  Word w of a (row tile, step) plane row covers k bytes 4w..4w+3 of
// the step: sub-chunk q = 4*step_in_chunk + w/4, channels 16*(q % cpt) + 4*(w%4)
// + 0..3 of the chunk, tap q / cpt.  Besides the two limb planes the row is
// written as int8 values (w8 plane: meaningful when every weight of the row
// lies in [-128, 127], which wfit records).  The weight loads are range-checked
// buffer loads (a padding position reads 0 through bit 31 of its offset: no
// branch between them), and the row sum and the int8 flag are wave reductions
// met in LDS after one barrier.
struct PackArgs {
    const int16_t* w;
    uint8_t* wpk;
    uint8_t* wpk8;
    uint32_t* wsum;
    uint32_t* wfit;
    uint32_t C, M, taps, nchunks, steps, steps_full;   // steps_full = taps (a full chunk)
    uint32_t tb;                                         // rows per row tile
};

__global__ __launch_bounds__(256) void conv_wpack(PackArgs a) {
    const uint32_t m = blockIdx.x;   // 0 .. Mpad-1
    const uint32_t mt = m / a.tb, r = m % a.tb;
    const uint32_t tile = 2u * a.tb * 64u, tile8 = a.tb * 64u;   // bytes per (row tile, step)
    const bool mok = m < a.M;
    const uint32_t row_elems = a.C * a.taps;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.w + (uint64_t)(mok ? m : 0u) * row_elems,
                                               mok ? row_elems * 2u : 0u);
    uint32_t sum = 0, fit = 1u;
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
        const uint32_t live = (uint32_t)(tap < a.taps);
        uint32_t v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t cl = cg * 16u + (wd & 3u) * 4u + j;
            const uint32_t ok = live & (uint32_t)(cl < cc);
            const uint32_t off = ((((c0 + cl) * a.taps + tap) * 2u) & 0x7FFFFFFFu) | ((ok ^ 1u) << 31);
            v[j] = (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
        }
        uint32_t hw = 0, lw = 0, bw = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int32_t x = (int32_t)(int16_t)v[j];
            sum += (uint32_t)x;
            fit &= (uint32_t)(x >= -128 && x <= 127);
            hw |= hi_byte(x) << (8 * j);
            lw |= lo_byte(x) << (8 * j);
            bw |= ((uint32_t)x & 0xFFu) << (8 * j);
        }
        uint8_t* dst = a.wpk + (uint64_t)(mt * a.steps + gs) * tile + r * 64u + wd * 4u;
        *reinterpret_cast<uint32_t*>(dst) = hw;
        *reinterpret_cast<uint32_t*>(dst + a.tb * 64u) = lw;
        *reinterpret_cast<uint32_t*>(a.wpk8 + (uint64_t)(mt * a.steps + gs) * tile8 + r * 64u + wd * 4u) = bw;
    }
    // row sum (every real weight once; padding adds 0) and the int8 flag: per
    // wave, then the four waves' values after one barrier
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += (uint32_t)__shfl_xor((int)sum, o, 64);
    const uint32_t wave_fit = __ballot(fit == 0u) == 0ull ? 1u : 0u;
    __shared__ uint32_t red[2][4];
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63u) == 0) {
        red[0][w] = sum;
        red[1][w] = wave_fit;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (mok) a.wsum[m] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
        a.wfit[m] = red[1][0] & red[1][1] & red[1][2] & red[1][3];
    }
}

// ------------------------------------------------------------- main kernel --
// Block: 256 threads = 4 waves as WR rows x 4/WR columns; a row tile of 32*WR
// output channels of one range of L consecutive output pixels of one image,
// computed in sub-tiles of 64*4/WR pixels; wave tile 32 channels x 64 pixels
// (2 x 4 MFMA 16x16x64 tiles, three accumulator sets).  Waves of one row read
// their own weight rows; waves of one column read their own 64 pixels of the
// patch.  (WR = 4 for more than 64 output channels, 2 for 33-64, 1 for <= 32.)
// When the LDS patch holds every channel, the input rows of the range are
// staged once and every sub-tile reads them; otherwise (MULTI) each sub-tile
// restages 64-channel chunks in turn.  After staging, each patch position's channel sum is
// kept in LDS, so a pixel's window sum (the limb identity's column sum) is a
// sum over taps, read outside the k loop.  A fragments come straight from the
// packed planes (a row tile of one limb is 16 rows x 64 bytes, 1 KB
// contiguous: one 16-byte load per lane), one step ahead, so the k loop has
// no barrier and no LDS writes.  Each wave finishes its own outputs through a
// private 16-row LDS tile (no block barrier) and stores rows of 8 pixels as
// 16-byte writes.
constexpr int kPgThreads = 256;
constexpr uint32_t kEpiPitch = 72;                      // int16 per row of a wave's epilogue tile
constexpr uint32_t kEpiBytes = 16u * kEpiPitch * 2u;    // 16 channel rows x 64 pixels (+ pad)
constexpr int kMaxTaps = kMaxQ / 4;

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// VEC: patch rows loaded 16 bytes at a time with g = VEC; 0 = per element.
// MULTI: 64-channel chunks restaged in turn inside the k loop (more channels
// than one patch holds), with fewer loads in flight while the accumulators are
// live.
// NS: A fragment sets in flight (3: two steps of prefetch, without MULTI and
// with a step count that is a multiple of 3; else 2: one step).
// WR: wave rows (row tile of 32 * WR output channels).
// PAIR: the block's outputs (every output channel: one row tile) feed a 1x1
// convolution in the same launch.  After a sub-tile's k loop the waves write
// the middle tensor (act1 applied) into LDS as limb planes, pixel-major (byte c
// of pixel px's row: channel c, the 1x1's k order), and after a barrier each
// wave computes 32 x 64 tiles of the 1x1 (A from its packed planes, B from the
// middle tile) and finishes them through the epilogue.
template <int VEC, bool MULTI, int NS, int WR, bool PAIR>
__global__ __launch_bounds__(kPgThreads, 2) void conv_pgemm(PgArgs g) {
    static_assert(NS == 2 || (NS == 3 && !MULTI), "three A sets need one patch of every channel");
    static_assert(!(PAIR && MULTI), "a pair needs one patch of every channel");
    constexpr uint32_t TB = 32u * WR;             // output channels per row tile
    constexpr uint32_t WC = 4u / WR;              // wave columns
    constexpr uint32_t SPX = 64u * WC;            // pixels per sub-tile
    constexpr uint32_t PT = 2u * TB * 64u;        // limb-plane bytes per (row tile, k step)
    constexpr uint32_t PT8 = TB * 64u;            // int8-plane bytes per (row tile, k step)
    constexpr int kPB = MULTI ? 1 : 4;   // 16-byte staging tasks per thread in flight
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int32_t qtab[kMaxQ + 4];  // per sub-chunk q: patch byte offset of its tap and group
    __shared__ uint32_t tpos[kMaxTaps];  // per tap: patch position offset from a window origin
    __shared__ uint32_t rowterm_s[kMaxTB];   // per output channel of the row tile: the row term
    __shared__ uint32_t flags_s[4];          // per wave: its rows' int8 votes
    uint8_t* p_hi = lds;
    uint8_t* p_lo = lds + g.p_plane;
    uint32_t* spos = reinterpret_cast<uint32_t*>(lds + g.spos_off);   // per position: channel sum

    // Touch every 64-byte line of the arguments at once: they arrive cold from
    // device memory, and fetched one at a time behind the branches that use
    // them they cost a memory round trip each.
    {
        uint32_t touch = 0;
#pragma unroll
        for (uint32_t i = 0; i < (sizeof(PgArgs) + 63) / 64; ++i)
            touch ^= reinterpret_cast<const uint32_t*>(&g)[i * 16];
        asm volatile("" ::"s"(touch));
    }
    const uint32_t tid = threadIdx.x;
    // the wave index in a scalar register: what derives from it (wave row and
    // column, tile coordinates, weight-row offsets) stays scalar too
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t lane = tid & 63;   // made opaque after each k loop (see there)
    int16_t* et = reinterpret_cast<int16_t*>(lds + g.epi_off + wave * kEpiBytes);
    // Workgroups are dealt to the 8 XCDs round robin; block b of XCD x takes the
    // x-th contiguous share of the (row tile, image, range) order, so ranges
    // that share input rows (and blocks that share weights) meet in one L2.
    const uint32_t nb = gridDim.x, per = nb >> 3, rem = nb & 7u, xcd = blockIdx.x & 7u, idx = blockIdx.x >> 3;
    const uint32_t lg = xcd < rem ? xcd * (per + 1u) + idx : rem * (per + 1u) + (xcd - rem) * per + idx;
    const uint32_t mt = fdiv(lg, g.div_nbm), rest = lg - mt * g.rpi_n;
    const uint32_t wr = wave / WC, wc = wave - wr * WC;   // the wave's row / column
    const uint32_t row0 = mt * TB, wrow = row0 + wr * 32;
    const uint32_t n = fdiv(rest, g.div_rpi);
    const uint32_t pb = (rest - n * g.rpi) * g.L;                       // the range's first pixel
    const uint32_t pe = min(pb + g.L, g.P);                             // one past its last
    const uint32_t oh_a = fdiv(pb, g.div_ow), oh_b = fdiv(pe - 1u, g.div_ow);
    const uint32_t prows_b = (oh_b - oh_a) * g.Sg + g.khspan;          // patch rows this range reads
    const int32_t ih_first = (int32_t)(oh_a * g.S) - (int32_t)g.pt;
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(g.x + (uint64_t)n * g.x_img, g.x_img_bytes);
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(reinterpret_cast<const int16_t*>(g.wpk), g.pk_bytes);
    const __amdgpu_buffer_rsrc_t wrs2 = make_rsrc(reinterpret_cast<const int16_t*>(g.wpk2), g.pk2_bytes);
    const uint32_t hw_in = g.H * g.W;

    if (tid == 0) {   // the zero slot: 16 bytes of each plane holding the limbs of 0
        *reinterpret_cast<v4u*>(p_hi + g.zslot) = v4u{0u, 0u, 0u, 0u};
        *reinterpret_cast<v4u*>(p_lo + g.zslot) = v4u{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
    }

    // A fragments of step gs: row tile i of the wave's 32 rows, hi and lo planes
    // (steps past the last one read another row tile's data or, past the buffer,
    // 0; neither is used)
    const uint32_t a_src = (mt * g.steps) * PT + (wr * 32u + (lane & 15)) * 64u + (lane >> 4) * 16u;
    auto a_load = [&](uint32_t gs, v4i (&ah)[2], v4i (&al)[2]) {
        const uint32_t off = a_src + gs * PT;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            ah[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wrs, off + i * 1024u, 0, 0));
            al[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                wrs, off + TB * 64u + i * 1024u, 0, 0));
        }
    };
    // the int8 plane's A fragments of step gs (rows whose weights all fit int8)
    const uint32_t a8_src = g.pk8_off + (mt * g.steps) * PT8 + (wr * 32u + (lane & 15)) * 64u +
                            (lane >> 4) * 16u;
    auto a_load8 = [&](uint32_t gs, v4i (&a8)[2]) {
        const uint32_t off = a8_src + gs * PT8;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            a8[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wrs, off + i * 1024u, 0, 0));
    };
    // Row terms and int8 flags of the block's 128 output channels: loaded here,
    // used after the patch is staged (128 * row sum + bias << 8)
    // (no bias: a buffer of range 0, whose loads read 0 -- `bias ? bias[r] : 0`
    // became a branch with a wait for every load issued before it, a memory
    // round trip ahead of the patch loads)
    const uint32_t rm = min(row0 + (tid & (TB - 1)), g.M - 1u);
    const uint32_t ld_wsum = g.wsum[rm], ld_fit = g.wfit[rm];
    const __amdgpu_buffer_rsrc_t brs = make_rsrc(g.bias ? g.bias : g.x, g.bias ? g.M * 2u : 0u);
    // (raw 16-bit values, sign-extended where the row terms are written: a
    // conversion here made the prologue wait for the load)
    const uint32_t ld_bias = __builtin_amdgcn_raw_buffer_load_b16(brs, rm * 2u, 0, 0);
    // PAIR: the 1x1's row terms and int8 flags (thread t: its row t), written
    // to LDS with the first conv's after the patch is staged; the middle tile's
    // bytes start as the limbs of 0 (k positions past the middle channels keep
    // them: the limb identity's zero operand)
    uint32_t ld_wsum2 = 0, ld_fit2 = 1u, ld_bias2 = 0;
    if constexpr (PAIR) {
        const uint32_t r2 = min(tid, g.M2 - 1u);
        ld_wsum2 = g.wsum2[r2];
        ld_fit2 = g.wfit2[r2];
        const __amdgpu_buffer_rsrc_t b2rs = make_rsrc(g.bias2 ? g.bias2 : g.x, g.bias2 ? g.M2 * 2u : 0u);
        ld_bias2 = __builtin_amdgcn_raw_buffer_load_b16(b2rs, r2 * 2u, 0, 0);
        const uint32_t nv = (SPX * g.HP + 64u) / 16u;   // a plane and its 64 padding bytes
        for (uint32_t v = tid; v < nv; v += kPgThreads) {
            *reinterpret_cast<v4u*>(lds + g.hp_off + v * 16u) = v4u{0u, 0u, 0u, 0u};
            *reinterpret_cast<v4u*>(lds + g.hp_off + SPX * g.HP + 64u + v * 16u) =
                v4u{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
        }
    }
    bool fast2 = true;   // PAIR: every 1x1 weight fits int8 (two limb products)

    // Patch staging of one chunk (the range's rows; tasks past prows_b are
    // skipped).  Rows outside the image and channels past C read 0 through the
    // buffer range.
    auto stage_patch = [&](uint32_t c0, uint32_t cpt) {
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
                    const uint32_t live = (uint32_t)(e < ntask) & (uint32_t)(r < prows_b);
                    const uint32_t okp = live & (uint32_t)((uint32_t)ih < g.H) & (uint32_t)((uint32_t)iw < g.W);
                    const uint32_t c = c0 + cq * 4u;
                    const uint32_t base = (c * hw_in + (uint32_t)ih * g.W + (uint32_t)iw) * 2u;
                    dst[u] = live ? pos * g.ppitch + cq * 4u : 0xFFFFFFFFu;
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
            // Each thread takes one (patch row r, 8-column group vv) pair and every
            // G-th channel quad from g0 (G = pair groups that fit the block), so a
            // task's addresses are the previous task's plus constant steps.
            const uint32_t nv = g.W / 8u;
            const uint32_t npr = g.prows * nv;
            const uint32_t G = g.stage_g;
            const uint32_t lh = (g.pl + VEC - 1u) / VEC;   // patch column of the first input column used
            const uint32_t plane2 = hw_in * 2u;             // bytes of one input channel plane
            const uint32_t src_step = G * 4u * plane2, dst_step = G * 4u;
            for (uint32_t v = tid; v < G * npr; v += kPgThreads) {
                const uint32_t g0 = fdiv(v, g.div_npr), pr = v - g0 * npr;
                const uint32_t r = fdiv(pr, g.div_nv), vv = pr - r * nv;
                if (r >= prows_b) continue;
                const int32_t ih = ih_first + (int32_t)(r * VEC);
                const uint32_t okr = (uint32_t)((uint32_t)ih < g.H);
                uint32_t src = ((c0 + g0 * 4u) * hw_in + (uint32_t)ih * g.W + vv * 8u) * 2u;
                uint32_t dst = (r * g.PW + vv * (8u / VEC) + lh) * g.ppitch + g0 * 4u;
                uint32_t c = c0 + g0 * 4u;
                for (uint32_t cq = g0; cq < ncq; cq += kPB * G) {
                v4u d[kPB][4];
#pragma unroll
                for (int u = 0; u < kPB; ++u) {
                    const uint32_t cu = c + u * 4u * G;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const uint32_t ok = okr & (uint32_t)(cu + jj < g.C) & (uint32_t)(cq + u * G < ncq);
                        const uint32_t off = ((src + u * src_step + jj * plane2) & 0x7FFFFFFFu) | ((ok ^ 1u) << 31);
                        d[u][jj] = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
                    }
                }
                uint32_t dst0[kPB];
#pragma unroll
                for (int u = 0; u < kPB; ++u) dst0[u] = dst + u * dst_step;
#pragma unroll
                for (int u = 0; u < kPB; ++u) {
                    if (cq + u * G >= ncq) continue;
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
                src += kPB * src_step;
                dst += kPB * dst_step;
                c += kPB * 4u * G;
                }
            }
            // padding columns (input columns outside the row) that a window reads:
            // left [0, lhc), right [wr, PWr)
            const uint32_t nhalo = ncq * g.prows * g.nh;
            for (uint32_t e = tid; e < nhalo; e += kPgThreads) {
                const uint32_t cqr = fdiv(e, g.div_nh), hcol = e - cqr * g.nh;
                const uint32_t cq = fdiv(cqr, g.div_prows), r = cqr - cq * g.prows;
                if (r >= prows_b) continue;
                const uint32_t col = hcol < g.lhc ? hcol : g.wr + (hcol - g.lhc);
                const uint32_t dst = (r * g.PW + col) * g.ppitch + cq * 4u;
                *reinterpret_cast<uint32_t*>(p_hi + dst) = 0u;
                *reinterpret_cast<uint32_t*>(p_lo + dst) = 0x80808080u;
            }
        }
    };

    // The q table of the staged patch (it depends on no loaded data, so it is
    // written before the patch loads land): sub-chunk q -> byte offset of its
    // (tap, 16-channel group) from a pixel's window origin, -1 past the last
    // sub-chunk.  The first nfull * taps * 4 entries walk full 64-channel chunks
    // (q = 4 * (chunk * taps + tap) + group), the rest the last chunk's cpt
    // groups (q = tap * cpt + group); with every chunk in one patch the groups
    // of chunk ch sit at slot 4 * ch + group of a position.
    auto build_qtab = [&](uint32_t cpt, const FastDiv& div_cpt, uint32_t nfull) {
        const uint32_t qfull = nfull * g.taps * 4u;
        for (uint32_t q = tid; q < (uint32_t)kMaxQ + 4u; q += kPgThreads) {
            uint32_t tap, cg;
            if (q < qfull) {
                const uint32_t ch = fdiv(q, g.div_t4), r = q - ch * g.taps * 4u;
                tap = r >> 2;
                cg = ch * 4u + (r & 3u);
            } else {
                const uint32_t r = q - qfull;
                tap = fdiv(r, div_cpt);
                cg = nfull * 4u + (r - tap * cpt);
            }
            const uint32_t khi = fdiv(tap, g.div_kw), kwi = tap - khi * g.KW;
            const uint32_t tp = (khi * g.PW + kwi) * g.Dg;
            qtab[q] = tap < g.taps ? (int32_t)(tp * g.ppitch + cg * 16u) : -1;
            if (q < (uint32_t)kMaxTaps) {
                const uint32_t kh2 = fdiv(q, g.div_kw), kw2 = q - kh2 * g.KW;
                tpos[q] = q < g.taps ? (kh2 * g.PW + kw2) * g.Dg : 0u;
            }
        }
    };
    // After a patch is staged: each position's sum over its cpt channel slots
    // (x = 256 * high + low + 128 per slot; a zero slot adds 0).
    auto pos_sums = [&](uint32_t cpt) {
        const uint32_t np = prows_b * g.PW;
        const uint32_t base = 128u * 16u * cpt;
        for (uint32_t pos = tid; pos < np; pos += kPgThreads) {
            int32_t sh = 0, sl = 0;
            for (uint32_t c = 0; c < cpt; ++c) {
                sh = bsum16(*reinterpret_cast<const v4i*>(p_hi + pos * g.ppitch + c * 16u), sh);
                sl = bsum16(*reinterpret_cast<const v4i*>(p_lo + pos * g.ppitch + c * 16u), sl);
            }
            spos[pos] = 256u * (uint32_t)sh + (uint32_t)sl + base;
        }
    };

    const uint32_t kp_term = 16384u * 64u * g.steps;
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    const bool plain = g.epi.add_mode == 0u && g.epi.act == 0u;   // no Add, no activation
    // The fused Add's operands of a 32-row tile (output rows m_base.., rows from
    // m_end on read 0; pixels p0w.. of the range, pnw of them valid), laid out as
    // finish_tile reads them (half i, run t: row (lane / 8) + 8t of the half,
    // pixels 8 * (lane % 8)..+8, as 8 packed int16), loaded ahead of the finish
    // in one go: 16-byte loads when the runs are 16-byte aligned, 4-byte loads
    // when they are 4-byte aligned, else 2-byte loads.  Values past a run's valid
    // pixels are never stored (they lie in the operand's image, or past it,
    // where the buffer reads 0); empty runs and rows past m_end read 0 through
    // bit 31 of their offset, never through a branch.  Every load is issued
    // before any is used.
    const __amdgpu_buffer_rsrc_t ars = make_rsrc(g.epi.add_mode == 1u ? g.epi.add + (uint64_t)n * g.y_img : g.x,
                                                 g.epi.add_mode == 1u ? (uint32_t)(g.y_img * 2u) : 0u);
    auto add_load = [&](uint32_t m_base, uint32_t m_end, uint32_t p0w, uint32_t pnw, v4u (&av)[2][2]) {
        const uint32_t c8 = (lane & 7) * 8;
        uint32_t off[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t m = m_base + i * 16 + (lane >> 3) + 8 * t;
                const uint32_t bad = (uint32_t)(m >= m_end || c8 >= pnw);
                off[i][t] = ((m * g.P + p0w + c8) * 2u) | (bad << 31);
            }
        if (g.vw == 8u) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int t = 0; t < 2; ++t) av[i][t] = __builtin_amdgcn_raw_buffer_load_b128(ars, off[i][t], 0, 0);
        } else if (g.add_w4) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        av[i][t][q] = __builtin_amdgcn_raw_buffer_load_b32(ars, off[i][t] + 4u * q, 0, 0);
        } else {
            uint32_t h[2][2][8];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        h[i][t][q] = __builtin_amdgcn_raw_buffer_load_b16(ars, off[i][t] + 2u * q, 0, 0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    av[i][t] = v4u{pack2(h[i][t][0], h[i][t][1]), pack2(h[i][t][2], h[i][t][3]),
                                   pack2(h[i][t][4], h[i][t][5]), pack2(h[i][t][6], h[i][t][7])};
        }
    };
    // Epilogue, per wave, of a 32-row x 64-pixel accumulator tile (output rows
    // m_base.., rows from m_end on skipped; pixels p0w.. of the range, pnw of them
    // valid, njw 16-pixel column tiles in use): each 16-row half is finished into
    // the wave's LDS tile (row 4*(lane/16)+e, pixel column of the lane), then read
    // back as 8-pixel runs: lane -> (row lane/8 + 8t, pixels 8*(lane%8)..)
    auto finish_tile = [&](const v4i (&th)[2][4], const v4i (&tm)[2][4], const v4i (&tl)[2][4],
                           uint32_t m_base, uint32_t m_end, uint32_t p0w, uint32_t pnw, uint32_t njw,
                           const v4u (&av)[2][2]) {
        const uint32_t c8 = (lane & 7) * 8;
        const uint32_t ncol = c8 < pnw ? min(8u, pnw - c8) : 0u;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if ((uint32_t)j >= njw) continue;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t v = ((uint32_t)th[i][j][e] << 16) + ((uint32_t)tm[i][j][e] << 8) +
                                       (uint32_t)tl[i][j][e];
                    et[((lane >> 4) * 4 + e) * kEpiPitch + j * 16 + (lane & 15)] = q88::acc_to_data(v);
                }
            }
            wave_sync();
            if (ncol) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint32_t r = (lane >> 3) + 8 * t;
                    const uint32_t m = m_base + i * 16 + r;
                    if (m >= m_end) continue;
                    const uint64_t o = (uint64_t)n * g.y_img + (uint64_t)m * g.P + p0w + c8;
                    const v4u tv = *reinterpret_cast<const v4u*>(et + r * kEpiPitch + c8);
                    int16_t* yp = g.y + o;
                    const bool vec8 = ncol == 8u && g.vw == 8u;
                    if (plain && vec8) {
                        *reinterpret_cast<v4u*>(yp) = tv;
                        continue;
                    }
                    int32_t yv[8];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        yv[2 * q] = (int32_t)(int16_t)(tv[q] & 0xFFFFu);
                        yv[2 * q + 1] = (int32_t)tv[q] >> 16;
                    }
                    if (g.epi.add_mode == 1u) {   // the operands add_load brought in
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            yv[2 * q] = q88::add(yv[2 * q], (int32_t)(int16_t)(av[i][t][q] & 0xFFFFu));
                            yv[2 * q + 1] = q88::add(yv[2 * q + 1], (int32_t)av[i][t][q] >> 16);
                        }
                    }
#pragma unroll
                    for (int q = 0; q < 8; ++q) yv[q] = q88::clamp(yv[q], lo, hi);
                    if (vec8) {
                        *reinterpret_cast<v4u*>(yp) = v4u{pack2(yv[0], yv[1]), pack2(yv[2], yv[3]),
                                                          pack2(yv[4], yv[5]), pack2(yv[6], yv[7])};
                    } else {
#pragma unroll
                        for (int q = 0; q < 8; ++q)
                            if ((uint32_t)q < ncol) yp[q] = (int16_t)yv[q];
                    }
                }
            }
            wave_sync();   // the tile's reads are done before the next half overwrites it
        }
    };
    const uint32_t nsub = (pe - pb + SPX - 1) / SPX;
    // A fragment sets: the set of global step gs is gs % NS, and the next NS - 1
    // steps' sets are in flight while a step's MFMAs run
    v4i fa_h[NS][2], fa_l[NS][2];
    uint32_t gs = 0;   // global k step of the next MFMA step, over all sub-tiles
    // every weight of the row tile fits int8: two limb products (w * x_hi and
    // w * x_lo) instead of four, and no column term
    bool fast = false;
    // step ks + d of a sub-tile, wrapping into the next sub-tile's steps
    auto ks_plus = [&](uint32_t ks, uint32_t d) {
        uint32_t k = ks + d;
        k = k >= g.steps ? k - g.steps : k;
        return k >= g.steps ? k - g.steps : k;
    };

    // The first steps' A fragments load before the patch, so their latency
    // overlaps the staging: the int8 form, which weights that fit int8 use
    // (known only once the block's flags are in; other weights reload the
    // limb planes then).
    a_load8(0, fa_h[0]);
    if constexpr (NS == 3) a_load8(ks_plus(0, 1), fa_h[1]);

    // The first chunk's patch (without MULTI: every chunk, staged once for every
    // sub-tile), before the accumulators of a sub-tile are live.  Without MULTI
    // this runs once ahead of the sub-tile loop: the staging loop's addresses then
    // die before the k loop instead of living (and being spilled) across it, and
    // their reloads cannot make the staging loads wait for the A fragments'.
    auto stage_first = [&](uint32_t sub) {
        if (sub) __syncthreads();   // every wave is done with the previous patch and q table
        stage_patch(0u, MULTI ? 4u : g.cpt_all);
        build_qtab(MULTI ? 4u : g.cpt_last, MULTI ? g.div_cpt4 : g.div_cpt_last, MULTI ? 0u : g.nfull);
        if (sub == 0) {
            // the prologue's loads are used from here on: the empty asm keeps
            // the compiler from computing with them (and so waiting for them)
            // ahead of the patch loads
            uint32_t wsum = ld_wsum, bias = ld_bias, fit = ld_fit;
            uint32_t wsum2 = ld_wsum2, bias2 = ld_bias2, fit2 = ld_fit2;
            asm volatile("" : "+v"(wsum), "+v"(bias), "+v"(fit), "+v"(wsum2), "+v"(bias2), "+v"(fit2));
            const bool real = row0 + tid < g.M;
            if (tid < TB) rowterm_s[tid] = real ? 128u * wsum + (uint32_t)(int32_t)(int16_t)bias * 256u : 0u;
            if constexpr (PAIR) {
                if (tid < ((g.M2 + 31u) & ~31u))
                    reinterpret_cast<uint32_t*>(lds + g.rt2_off)[tid] =
                        tid < g.M2 ? 128u * wsum2 + (uint32_t)(int32_t)(int16_t)bias2 * 256u : 0u;
            }
            // the int8 flags: a wave vote each, met in LDS behind the one barrier
            // the patch needs anyway (bit 0: a row of the tile past int8, bit 1:
            // a 1x1 row past int8)
            const bool wide1 = tid < TB && real && fit == 0u;
            const bool wide2 = PAIR && tid < g.M2 && fit2 == 0u;
            const uint32_t vote = (__ballot(wide1) != 0ull ? 1u : 0u) | (__ballot(wide2) != 0ull ? 2u : 0u);
            if (lane == 0) flags_s[wave] = vote;
            __syncthreads();
            const uint32_t wide = __builtin_amdgcn_readfirstlane(flags_s[0] | flags_s[1] | flags_s[2] | flags_s[3]);
            fast = (wide & 1u) == 0u;
            fast2 = (wide & 2u) == 0u;
            if (!fast) {
                a_load(0, fa_h[0], fa_l[0]);
                if constexpr (NS == 3) a_load(ks_plus(0, 1), fa_h[1], fa_l[1]);
            }
        } else {
            __syncthreads();
        }
        if (!fast) {   // the column term's position sums
            pos_sums(MULTI ? 4u : g.cpt_all);
            __syncthreads();
        }
    };
    if constexpr (!MULTI) stage_first(0u);

    for (uint32_t sub = 0; sub < nsub; ++sub) {
        const uint32_t p0 = pb + sub * SPX + wc * 64u;      // this wave's first pixel of the sub-tile
        const uint32_t pn = p0 < pe ? min(64u, pe - p0) : 0u;   // the wave's pixels of this sub-tile
        const uint32_t nj = (pn + 15u) / 16u;              // 16-pixel column tiles in use (0 - 4)
        if constexpr (MULTI) stage_first(sub);
        // patch position of the window origin of this lane's pixel in each column
        // tile (row (oh - oh_a) * S', column ow * S') and its byte offset
        uint32_t ppos[4], pbase[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t px = min(p0 + j * 16 + (lane & 15), pe - 1u);   // past the range: any of its pixels
            const uint32_t oh = fdiv(px, g.div_ow), ow = px - oh * g.OW;
            ppos[j] = ((oh - oh_a) * g.PW + ow) * g.Sg;
            pbase[j] = ppos[j] * g.ppitch;
        }
        // accumulators: the low set starts at the row and constant terms; each
        // chunk adds 128 * its window sums (the column term)
        v4i hh[2][4], mid[2][4], ll[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                hh[i][j] = v4i{0, 0, 0, 0};
                mid[i][j] = v4i{0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ll[i][j][e] = (int32_t)(rowterm_s[wr * 32 + i * 16 + (lane >> 4) * 4 + e] - (fast ? 0u : kp_term));
            }
        auto window_sums = [&]() {
            uint32_t cs[4] = {0u, 0u, 0u, 0u};
            for (uint32_t t = 0; t < g.taps; ++t) {
                const uint32_t tp = tpos[t];
#pragma unroll
                for (int j = 0; j < 4; ++j) cs[j] += spos[ppos[j] + tp];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) ll[i][j][e] = (int32_t)((uint32_t)ll[i][j][e] + 128u * cs[j]);
        };

        // k loop over the chunks.  Software pipeline: the B fragments of column
        // tile j + 1 (of the next step's tile 0 after tile 3) are read from the
        // patch while tile j's MFMAs run, and the A fragments NS - 1 steps ahead
        // load while a step runs.  FULL: all four column tiles in use.  FAST:
        // int8 weights, sum w*x = 256 * sum w*x_hi + sum w*x_lo + 128 * sum w
        // (the last term is in the row term): mid gathers w*x_hi, ll w*x_lo.
        auto k_loop = [&](auto full, auto fastc) {
            constexpr bool FULL = decltype(full)::value;
            constexpr bool FAST = decltype(fastc)::value;
            v4i bh[2], bl[2];
            auto b_load = [&](int32_t qo, int j, v4i& h, v4i& l) {
                // past the chunk's last sub-chunk: the zero slot (the limbs of 0)
                const uint32_t a = qo >= 0 ? pbase[j] + (uint32_t)qo : g.zslot;
                h = *reinterpret_cast<const v4i*>(p_hi + a);
                l = *reinterpret_cast<const v4i*>(p_lo + a);
            };
            auto mfma_tile = [&](int j, const v4i& b_h, const v4i& b_l, const v4i (&ah)[2], const v4i (&al)[2]) {
                if constexpr (FAST) {
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], b_h, mid[i][j], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        ll[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], b_l, ll[i][j], 0, 0, 0);
                    return;
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    hh[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], b_h, hh[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], b_l, mid[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    ll[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], b_l, ll[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], b_h, mid[i][j], 0, 0, 0);
            };
            // one step with A set S.  FULL: on entry bh[0] / bl[0] hold tile 0 of
            // this step, and tile 3 prefetches the next step's tile 0; otherwise
            // the step reads its own tile 0 first.
            auto step = [&](auto set, uint32_t ls, uint32_t ks, int32_t& qo) {
                constexpr int S = decltype(set)::value;
                constexpr int SL = (S + NS - 1) % NS;   // the set of step ks + NS - 1
                if constexpr (FAST) a_load8(ks_plus(ks, NS - 1), fa_h[SL]);
                else a_load(ks_plus(ks, NS - 1), fa_h[SL], fa_l[SL]);
                const int32_t qn = qtab[(ls + 1u) * 4u + (lane >> 4)];   // next step's sub-chunk
                if constexpr (!FULL) b_load(qo, 0, bh[0], bl[0]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (!FULL && (uint32_t)j >= nj) continue;
                    const int jn = j + 1;
                    if constexpr (FULL) {
                        if (jn < 4) b_load(qo, jn, bh[jn & 1], bl[jn & 1]);
                        else b_load(qn, 0, bh[0], bl[0]);
                    } else {
                        if (jn < 4 && (uint32_t)jn < nj) b_load(qo, jn, bh[jn & 1], bl[jn & 1]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    mfma_tile(j, bh[j & 1], bl[j & 1], fa_h[S], fa_l[S]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                qo = qn;
            };
            uint32_t ks = 0;   // k step within this sub-tile
            for (uint32_t ch = 0; ch < (MULTI ? g.nchunks : 1u); ++ch) {
                const uint32_t c0 = ch * 64u;
                const bool last = ch + 1 == g.nchunks;
                const uint32_t cpt = last ? g.cpt_last : 4u;
                // without MULTI the one patch holds every chunk: all steps
                const uint32_t nst = MULTI ? (g.taps * cpt + 3u) / 4u : g.steps;
                if (MULTI && ch) {   // later chunks: restaged here
                    __syncthreads();   // every wave is done with the previous chunk's patch and q table
                    stage_patch(c0, cpt);
                    build_qtab(cpt, last ? g.div_cpt_last : g.div_cpt4, 0u);
                    __syncthreads();
                    if constexpr (!FAST) {
                        pos_sums(cpt);
                        __syncthreads();
                    }
                }
                if constexpr (!FAST) window_sums();
                int32_t qo = qtab[lane >> 4];
                if constexpr (FULL) b_load(qo, 0, bh[0], bl[0]);
                using S0 = std::integral_constant<int, 0>;
                using S1 = std::integral_constant<int, 1>;
                if constexpr (NS == 3) {   // every sub-tile starts at set 0 (steps % 3 == 0)
                    for (uint32_t ls = 0; ls < nst; ls += 3, gs += 3, ks += 3) {
                        step(S0{}, ls, ks, qo);
                        step(S1{}, ls + 1, ks + 1, qo);
                        step(std::integral_constant<int, 2>{}, ls + 2, ks + 2, qo);
                    }
                } else {
                    uint32_t ls = 0;
                    if (gs & 1u) {
                        step(S1{}, ls, ks, qo);
                        ++ls; ++gs; ++ks;
                    }
                    for (; ls + 2 <= nst; ls += 2, gs += 2, ks += 2) {
                        step(S0{}, ls, ks, qo);
                        step(S1{}, ls + 1, ks + 1, qo);
                    }
                    if (ls < nst) {
                        step(S0{}, ls, ks, qo);
                        ++gs; ++ks;
                    }
                }
            }
        };
        if (fast) {
            if (nj == 4u) k_loop(std::true_type{}, std::true_type{});
            else k_loop(std::false_type{}, std::true_type{});
        } else {
            if (nj == 4u) k_loop(std::true_type{}, std::false_type{});
            else k_loop(std::false_type{}, std::false_type{});
        }
        // Everything below recomputes its lane-dependent addresses: hoisted ahead
        // of the k loop they would hold registers across it (and be spilled, and
        // their reloads would wait for the loads issued after the k loop).
        asm volatile("" : "+v"(lane));

        if constexpr (!PAIR) {
            v4u av[2][2] = {};
            if (g.epi.add_mode == 1u) add_load(wrow, g.M, p0, pn, av);
            finish_tile(hh, mid, ll, wrow, g.M, p0, pn, nj, av);
        } else {
            // The 1x1: 32 x 64 tiles (row tile rt of its outputs, wave column cw's
            // pixels) dealt over the waves.  A tile's A fragments (both k steps;
            // with one step the second reads data that is never used) and its
            // fused-Add operands load ahead: the wave's first tile's here, before
            // the middle tile is written, the next tile's after a tile is finished.
            // ah2 comes from the int8 plane when every weight fits int8 (fast2,
            // chosen by a mask: no branch), else from the high limb plane; al2
            // always from the low limb plane (unused with fast2: copying ah2 into
            // it would wait for the load).
            const uint32_t nrt2 = (g.M2 + 31u) / 32u;
            const uint32_t arow = (lane & 15) * 64u + (lane >> 4) * 16u;
            v4i ah2[2][2], al2[2][2];
            v4u av2[2][2] = {};
            auto tile2 = [&](uint32_t t, uint32_t& rt, uint32_t& p0w, uint32_t& pnw) {
                rt = t / WC;
                const uint32_t cw = t - rt * WC;
                p0w = pb + sub * SPX + cw * 64u;
                pnw = p0w < pe ? min(64u, pe - p0w) : 0u;
            };
            const uint32_t f2mask = fast2 ? ~0u : 0u;
            auto load2 = [&](uint32_t t) {
                uint32_t rt, p0w, pnw;
                tile2(t, rt, p0w, pnw);
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) {
                    const uint32_t ro = rt * g.steps2 + (uint32_t)s2;
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const uint32_t oh = ro * 4096u + i * 1024u + arow;
                        const uint32_t o8 = g.pk2_8off + ro * 2048u + i * 1024u + arow;
                        ah2[s2][i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                                                 wrs2, oh ^ ((oh ^ o8) & f2mask), 0, 0));
                        al2[s2][i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                                                 wrs2, oh + 2048u, 0, 0));
                    }
                }
                if (g.epi.add_mode == 1u) add_load(rt * 32u, g.M2, p0w, pnw, av2);
            };
            if (wave < nrt2 * WC) load2(wave);
            // the middle tensor of this sub-tile, act1(sat16(acc >> 8)), as limb
            // planes: pixel px of the sub-tile at px * HP, channel c at byte c
            // (rows past the middle channels hold 0: their weights are 0)
            uint8_t* h_hi = lds + g.hp_off;
            uint8_t* h_lo = h_hi + SPX * g.HP + 64u;
            const int32_t lo1 = q88::act_lo(g.act1), hi1 = q88::act_hi(g.act1);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t hw = 0, lw = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t v = ((uint32_t)hh[i][j][e] << 16) + ((uint32_t)mid[i][j][e] << 8) +
                                           (uint32_t)ll[i][j][e];
                        const int32_t d = q88::clamp((int32_t)q88::acc_to_data(v), lo1, hi1);
                        hw |= hi_byte(d) << (8 * e);
                        lw |= lo_byte(d) << (8 * e);
                    }
                    const uint32_t a = (wc * 64u + j * 16u + (lane & 15)) * g.HP + wr * 32u + i * 16u +
                                       (lane >> 4) * 4u;
                    *reinterpret_cast<uint32_t*>(h_hi + a) = hw;
                    *reinterpret_cast<uint32_t*>(h_lo + a) = lw;
                }
            __syncthreads();
            // four limb products: each pixel's sum over the 1x1's k positions
            uint32_t* cs = reinterpret_cast<uint32_t*>(lds + g.cs_off);
            if (!fast2) {
                for (uint32_t px = tid; px < SPX; px += kPgThreads) {
                    int32_t sh = 0, sl = 0;
                    for (uint32_t c = 0; c < g.steps2 * 4u; ++c) {
                        sh = bsum16(*reinterpret_cast<const v4i*>(h_hi + px * g.HP + c * 16u), sh);
                        sl = bsum16(*reinterpret_cast<const v4i*>(h_lo + px * g.HP + c * 16u), sl);
                    }
                    cs[px] = 256u * (uint32_t)sh + (uint32_t)sl + 128u * 64u * g.steps2;
                }
                __syncthreads();
            }
            const uint32_t* rt2 = reinterpret_cast<const uint32_t*>(lds + g.rt2_off);
            const uint32_t kp2 = fast2 ? 0u : 16384u * 64u * g.steps2;
            for (uint32_t t = wave; t < nrt2 * WC; t += 4u) {
                uint32_t rt, p0w, pnw;
                tile2(t, rt, p0w, pnw);
                if (pnw != 0u) {
                    const uint32_t cw = t - rt * WC;
                    const uint32_t njw = (pnw + 15u) / 16u;
                    v4i h2[2][4], m2[2][4], l2[2][4];
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            h2[i][j] = v4i{0, 0, 0, 0};
                            m2[i][j] = v4i{0, 0, 0, 0};
                            const uint32_t colt = fast2 ? 0u : 128u * cs[cw * 64u + j * 16u + (lane & 15)];
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                l2[i][j][e] = (int32_t)(rt2[rt * 32u + i * 16u + (lane >> 4) * 4u + e] - kp2 + colt);
                        }
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2) {
                        if ((uint32_t)s2 >= g.steps2) continue;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            if ((uint32_t)j >= njw) continue;
                            const uint32_t b = (cw * 64u + j * 16u + (lane & 15)) * g.HP + s2 * 64u + (lane >> 4) * 16u;
                            const v4i bh = *reinterpret_cast<const v4i*>(h_hi + b);
                            const v4i bl = *reinterpret_cast<const v4i*>(h_lo + b);
                            if (fast2) {   // sum w*x = 256 * sum w*x_hi + sum w*x_lo + 128 * sum w
#pragma unroll
                                for (int i = 0; i < 2; ++i) {
                                    m2[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah2[s2][i], bh, m2[i][j], 0, 0, 0);
                                    l2[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah2[s2][i], bl, l2[i][j], 0, 0, 0);
                                }
                            } else {
#pragma unroll
                                for (int i = 0; i < 2; ++i) {
                                    h2[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah2[s2][i], bh, h2[i][j], 0, 0, 0);
                                    m2[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah2[s2][i], bl, m2[i][j], 0, 0, 0);
                                    l2[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al2[s2][i], bl, l2[i][j], 0, 0, 0);
                                    m2[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al2[s2][i], bh, m2[i][j], 0, 0, 0);
                                }
                            }
                        }
                    }
                    finish_tile(h2, m2, l2, rt * 32u, g.M2, p0w, pnw, njw, av2);
                }
                if (t + 4u < nrt2 * WC) load2(t + 4u);
            }
            if (sub + 1 < nsub) __syncthreads();   // the next sub-tile's middle tile overwrites this one
        }
    }
}

inline bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

uint32_t gcd(uint32_t a, uint32_t b) {
    while (b) { const uint32_t t = a % b; a = b; b = t; }
    return a;
}

// Compute units of the current device (256 on MI355X), cached per device.
uint32_t cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256u;
    }
    int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return (uint32_t)c;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) {
        (void)hipGetLastError();
        c = 256;
    }
    cache[dev].store(c, std::memory_order_relaxed);
    return (uint32_t)c;
}

constexpr uint64_t kPgLdsMax = 78u * 1024u;   // dynamic LDS per block: two blocks per CU

}  // namespace

uint32_t cm_cu_count() { return cu_count(); }

namespace {

enum PgMode { kPackAndRun, kPackOnly, kRunPacked };

// A 1x1 convolution fused after the patch GEMM (the pair path): its weights
// [out_ch][mid] (mid = the first convolution's output channels), bias, and the
// activation applied to the middle tensor.
struct PairSpec {
    const int16_t* w2;
    const int16_t* bias2;
    uint32_t out_ch;
    uint32_t act1;
};
constexpr uint32_t kPairMaxOut = 256;   // the 1x1's output channels: one per thread for its row terms

// One patch-GEMM call: pack the weights into lc.ws and run (kPackAndRun), only
// pack them into `dst` (kPackOnly), or run with weights packed earlier
// (kRunPacked, `packed`).  Returns 1 (launching nothing) when the shape does
// not suit this path or the workspace is too small; with lc.need set, records
// the bytes the packed weights take.
int pg_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y, uint32_t batch,
              uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h,
              uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t sh, uint32_t sw, uint32_t dh,
              uint32_t dw, uint32_t pad_top, uint32_t pad_left, const cm_epilogue_t* epi,
              const LaunchCtx& lc, PgMode mode, const void* packed, void* dst, size_t dst_bytes,
              const PairSpec* pair = nullptr) {
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
    const uint32_t nchunks = (in_ch + 63) / 64;
    // row tile: 32, 64 or 128 output channels (128 with several channel chunks)
    const uint32_t wrows = nchunks > 1 || out_ch > 64 ? 4u : out_ch > 32 ? 2u : 1u;
    const uint32_t TB = 32u * wrows, SPX = 256u / wrows;
    const uint32_t mtiles = (out_ch + TB - 1) / TB;
    const uint32_t gg = gcd(sh, dh), Sg = sh / gg, Dg = dh / gg;
    if ((uint64_t)out_ch * P * 2 >= 0x80000000ull) return 1;
    // pair: one row tile holds every middle channel; the 1x1's k steps (64
    // channels each, at most two) and its LDS: the middle tile's two planes,
    // pixel column sums and row terms.  HP, the bytes per pixel, is an odd
    // multiple of 16 with room for the TB channels the waves write: 48 for a
    // 32-row tile (the 1x1's one k step then reads 16 bytes of the next pixel:
    // k positions whose weights are 0, read alike by the MFMAs and the column
    // sums, so the limb identity stays exact), else the k bytes + 16 (80 or
    // 144).  Each plane ends in 64 bytes of the limbs of 0, which the last
    // pixel's read reaches.
    const uint32_t m2 = pair ? pair->out_ch : 0u;
    const uint32_t steps2 = pair ? (out_ch + 63u) / 64u : 0u;
    const uint32_t HP = !pair ? 0u : TB == 32u ? 48u : std::max(steps2 * 64u, TB) + 16u;
    if (pair && (mtiles != 1u || m2 == 0u || m2 > kPairMaxOut || pair->act1 > 2u ||
                 (uint64_t)m2 * P * 2 >= 0x80000000ull))
        return 1;
    uint64_t pair_lds = pair ? 2ull * (SPX * HP + 64u) + 4ull * SPX + 4ull * kPairMaxOut : 0u;
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
    const uint32_t khspan = (kh - 1) * Dg + 1;
    const uint32_t last_cpt = (in_ch - (nchunks - 1) * 64 + 15) / 16;
    const uint32_t cpt_all = (in_ch + 15) / 16;
    uint32_t steps = (nchunks - 1) * taps + (taps * last_cpt + 3) / 4;
    auto a16 = [](uint64_t v) { return (v + 15) & ~15ull; };
    // LDS bytes per patch position and plane: an odd multiple of 16 (the 16
    // pixels of a fragment read then fall on distinct bank groups)
    auto pitch_of = [](uint32_t cpt) { return cpt % 2 ? cpt * 16 : cpt * 16 + 16; };
    auto layout = [&](uint64_t prows, uint32_t pitch, uint64_t& spos_off, uint64_t& epi_off) {
        const uint64_t p_plane = prows * PW * pitch + 16;
        spos_off = a16(2 * p_plane);
        epi_off = spos_off + a16(prows * PW * 4);
        return epi_off + 4ull * kEpiBytes + pair_lds;
    };
    // Pixels per block L (a multiple of 16): the fewest modelled cycles per CU,
    // with blocks dealt over the CUs two at a time.  A wave's 16-pixel column
    // tile costs 128 MFMA cycles per k step, and a block takes as long as its
    // busiest wave (sub-tiles of 64 pixels per wave column); staging a patch
    // row costs about one cycle per 16 bytes loaded, once per block pair (the
    // second block's staging overlaps the first one's MFMAs) and once per
    // sub-tile and chunk when chunks are restaged; a lone block per CU keeps
    // one wave per SIMD and runs at about 70%.  Returns 0 when no L fits.
    const uint64_t cus = cu_count();
    const uint64_t c_tile = 128ull * steps;
    auto pick_l = [&](bool multi, uint32_t pitch, uint64_t& prows_out) -> uint32_t {
        const uint32_t cpt_row = multi ? 4u : cpt_all;
        const uint64_t c_row = (uint64_t)PW * cpt_row * 2;
        uint32_t l_best = 0;
        uint64_t best = ~0ull;
        const uint64_t lcap = multi ? 128u : 512u;
        for (uint64_t l = 16; l <= lcap; l += 16) {
            // output rows a range spans: ranges start at multiples of l, so a
            // range's offset within its first row is a multiple of gcd(l, out_w),
            // at most out_w - gcd(l, out_w)
            const uint64_t off = out_w - gcd((uint32_t)l, out_w);
            const uint64_t rows = std::min<uint64_t>(out_h, (off + l + out_w - 1) / out_w);
            const uint64_t pr = (rows - 1) * Sg + khspan;
            uint64_t so, eo;
            // (rows do not grow monotonically with l: a longer, row-aligned range
            // may span fewer rows than a shorter one)
            if (layout(pr, pitch, so, eo) > kPgLdsMax) continue;
            const uint64_t rpi = (P + l - 1) / l;
            const uint64_t blocks = rpi * batch * mtiles;
            if (blocks > 0x7FFFFFFFull) continue;
            const uint64_t k = (blocks + cus - 1) / cus;
            const uint64_t rem = l % SPX;
            const uint64_t u = (l / SPX) * 4 + (std::min<uint64_t>(rem, 64) + 15) / 16;
            const uint64_t stage = pr * c_row * (multi ? nchunks * ((l + SPX - 1) / SPX) : 1u);
            uint64_t t = k * u * c_tile + ((k + 1) / 2) * stage;
            if (k == 1) t = t * 10 / 7;
            if (t < best) { best = t; l_best = (uint32_t)l; prows_out = pr; }
            if (l >= P) break;
        }
        return l_best;
    };
    // Every channel chunk staged once into one patch when the patch fits and the
    // q table holds every step; otherwise (MULTI) 64-channel chunks restaged in
    // turn.  Both consume the same packed weights (the k order is the chunk's).
    uint64_t prows = 0;
    uint32_t ppitch = pitch_of(cpt_all);
    bool multi = false;
    uint32_t L = steps * 4u <= (uint32_t)kMaxQ ? pick_l(false, ppitch, prows) : 0u;
    if (pair && L) {
        // the middle tile's LDS must not cost the pair more than half of the
        // pixel range the convolution alone would take (shorter ranges re-stage
        // more halo rows in more blocks than the saved launch is worth)
        const uint64_t keep = pair_lds;
        uint64_t pr0 = 0;
        pair_lds = 0;
        const uint32_t L0 = pick_l(false, ppitch, pr0);
        pair_lds = keep;
        if (2u * L < L0) return 1;
    }
    if (L == 0 && nchunks > 1 && !pair) {
        multi = true;
        ppitch = pitch_of(4u);
        L = pick_l(true, ppitch, prows);
    }
    if (L == 0) return 1;
    // With one patch of every chunk, a step count padded to a multiple of 3
    // (k steps of zero weights, which the pack writes as the limbs of 0 and the
    // q table sends to the zero slot: both sides of the limb identity gain
    // 16384 per position, or nothing on the int8 path) runs the three-set
    // pipeline, two steps of A fragments in flight instead of one; worth it
    // when the added steps are at most an eighth of the real ones.
    if (!multi) {
        const uint32_t pad = (3u - steps % 3u) % 3u;
        if (pad && 8u * pad <= steps && (steps + pad) * 4u <= (uint32_t)kMaxQ) steps += pad;
    }
    uint64_t spos_off = 0, epi_off = 0;
    const uint64_t lds = layout(prows, ppitch, spos_off, epi_off);
    const uint32_t rpi = (uint32_t)((P + L - 1) / L);
    const uint64_t zslot = prows * PW * ppitch;
    const uint64_t p_plane = zslot + 16;
    // workspace: limb planes, int8 plane, row sums, int8 flags
    const uint64_t pk_limb = (uint64_t)mtiles * steps * (2u * TB * 64u);
    const uint64_t pk_bytes = pk_limb + (uint64_t)mtiles * steps * (TB * 64u);
    // pair: the 1x1's packed weights after the first convolution's (32-row
    // tiles, the same plane layout with one tap), then its row sums and flags
    const uint32_t mtiles2 = (m2 + 31u) / 32u;
    const uint64_t off2 = pair ? (pk_bytes + 8ull * mtiles * TB + 255u) & ~255ull : 0u;
    const uint64_t pk2_limb = (uint64_t)mtiles2 * steps2 * (2u * 32u * 64u);
    const uint64_t pk2_bytes = pk2_limb + (uint64_t)mtiles2 * steps2 * (32u * 64u);
    const uint64_t need = pair ? off2 + pk2_bytes + 8ull * mtiles2 * 32u : pk_bytes + 8ull * mtiles * TB;
    if (pk_bytes >= 0x80000000ull) return 1;
    if (lc.need) {
        if (need > *lc.need) *lc.need = need;
        return CM_OK;
    }
    uint8_t* wbuf = nullptr;
    if (mode == kRunPacked) {
        if (!packed || !aligned(packed, 16)) return cm_set_error(CM_ERR_INVALID, "conv packed: weights not 16-byte aligned");
    } else {
        wbuf = static_cast<uint8_t*>(mode == kPackOnly ? dst : lc.ws);
        const size_t have = mode == kPackOnly ? dst_bytes : lc.ws_bytes;
        if (!wbuf || have < need || !aligned(wbuf, 16)) {
            if (mode == kPackOnly)
                return cm_set_error(CM_ERR_RANGE, "conv pack: %zu bytes given, %llu needed", have,
                                    (unsigned long long)need);
            return 1;
        }
        PackArgs pa{w, wbuf, wbuf + pk_limb, reinterpret_cast<uint32_t*>(wbuf + pk_bytes),
                    reinterpret_cast<uint32_t*>(wbuf + pk_bytes) + mtiles * TB,
                    in_ch, out_ch, taps, nchunks, steps, taps, TB};
        hipLaunchKernelGGL(conv_wpack, dim3(mtiles * TB), dim3(256), 0, lc.s, pa);
        int rc = cm_check_launch("conv_wpack");
        if (!rc && pair) {
            uint8_t* w2 = wbuf + off2;
            PackArgs pb2{pair->w2, w2, w2 + pk2_limb, reinterpret_cast<uint32_t*>(w2 + pk2_bytes),
                         reinterpret_cast<uint32_t*>(w2 + pk2_bytes) + mtiles2 * 32u,
                         out_ch, m2, 1u, steps2, steps2, 1u, 32u};
            hipLaunchKernelGGL(conv_wpack, dim3(mtiles2 * 32u), dim3(256), 0, lc.s, pb2);
            rc = cm_check_launch("conv_wpack");
        }
        if (rc || mode == kPackOnly) return rc;
    }
    const uint8_t* wpk = mode == kRunPacked ? static_cast<const uint8_t*>(packed) : wbuf;
    const uint32_t* wsum = reinterpret_cast<const uint32_t*>(wpk + pk_bytes);
    const uint32_t* wfit = wsum + mtiles * TB;

    PgArgs g{};
    g.x = x; g.wpk = wpk; g.wsum = wsum; g.wfit = wfit; g.bias = bias; g.y = y;
    g.C = in_ch; g.H = in_h; g.W = in_w; g.M = out_ch; g.OH = out_h; g.OW = out_w; g.P = (uint32_t)P;
    g.KW = kw; g.taps = taps; g.S = sh; g.Sg = Sg; g.Dg = Dg; g.g = gg; g.pt = pad_top; g.pl = pad_left;
    g.khspan = khspan;
    g.nchunks = nchunks; g.steps = steps;
    g.PW = PW; g.ppitch = ppitch; g.p_plane = (uint32_t)p_plane; g.zslot = (uint32_t)zslot;
    g.spos_off = (uint32_t)spos_off; g.epi_off = (uint32_t)epi_off;
    g.lhc = lhc; g.wr = wr; g.nh = nh;
    g.cpt_last = last_cpt;
    g.cpt_all = cpt_all;
    g.nfull = nchunks - 1;
    g.L = L; g.rpi = rpi; g.rpi_n = rpi * batch;
    g.div_nbm = make_fastdiv(rpi * batch);
    g.prows = (uint32_t)prows;
    g.npos = (uint32_t)prows * PW;
    g.div_rpi = make_fastdiv(rpi);
    g.div_ow = make_fastdiv(out_w);
    g.div_npos = make_fastdiv(g.npos);
    g.div_pw = make_fastdiv(PW);
    g.div_nv = make_fastdiv(in_w / 8 ? in_w / 8 : 1);
    {
        const uint32_t npr = (uint32_t)prows * (in_w / 8 ? in_w / 8 : 1);
        g.stage_g = npr < kPgThreads ? kPgThreads / npr : 1u;
        g.div_npr = make_fastdiv(npr);
    }
    g.div_prows = make_fastdiv((uint32_t)prows);
    g.div_nh = make_fastdiv(nh ? nh : 1);
    g.div_kw = make_fastdiv(kw);
    g.div_cpt4 = make_fastdiv(4);
    g.div_cpt_last = make_fastdiv(last_cpt);
    g.div_t4 = make_fastdiv(taps * 4u);
    g.x_img_bytes = (uint32_t)(2 * x_img);
    g.pk_bytes = (uint32_t)pk_bytes;
    g.pk8_off = (uint32_t)pk_limb;
    g.x_img = x_img;
    g.y_img = (uint64_t)(pair ? m2 : out_ch) * P;
    g.epi = ea;
    if (pair) {
        const uint8_t* w2 = wpk + off2;
        g.wpk2 = w2;
        g.wsum2 = reinterpret_cast<const uint32_t*>(w2 + pk2_bytes);
        g.wfit2 = g.wsum2 + mtiles2 * 32u;
        g.bias2 = pair->bias2;
        g.M2 = m2; g.steps2 = steps2; g.HP = HP;
        g.hp_off = (uint32_t)(epi_off + 4ull * kEpiBytes);
        g.cs_off = g.hp_off + 2u * (SPX * HP + 64u);
        g.rt2_off = g.cs_off + 4u * SPX;
        g.pk2_bytes = (uint32_t)pk2_bytes;
        g.pk2_8off = (uint32_t)pk2_limb;
        g.act1 = pair->act1;
    }
    // 16-byte output accesses: every run of 8 pixels starts 16-byte aligned
    // (ranges start at multiples of L, sub-tiles at multiples of 64 pixels)
    g.vw = P % 8 == 0 && aligned(y, 16) && (ea.add_mode != 1u || aligned(ea.add, 16)) ? 8u : 1u;
    g.add_w4 = P % 2 == 0 && ea.add_mode == 1u && aligned(ea.add, 4) ? 1u : 0u;
    const void* k = nullptr;
#define CM_PG_PICK(M, NS, W, PR) (vec == 1 ? (const void*)conv_pgemm<1, M, NS, W, PR> \
                                  : vec == 2 ? (const void*)conv_pgemm<2, M, NS, W, PR> \
                                             : (const void*)conv_pgemm<0, M, NS, W, PR>)
#define CM_PG_PICK_W(M, NS, PR) (wrows == 1 ? CM_PG_PICK(M, NS, 1, PR) : wrows == 2 ? CM_PG_PICK(M, NS, 2, PR) \
                                                                             : CM_PG_PICK(M, NS, 4, PR))
    if (multi) k = CM_PG_PICK(true, 2, 4, false);
    else if (pair) k = steps % 3 == 0 ? CM_PG_PICK_W(false, 3, true) : CM_PG_PICK_W(false, 2, true);
    else if (steps % 3 == 0) k = CM_PG_PICK_W(false, 3, false);
    else k = CM_PG_PICK_W(false, 2, false);
#undef CM_PG_PICK_W
#undef CM_PG_PICK
    if (lds > 65536u &&
        hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
        (void)hipGetLastError();
        return cm_set_error(CM_ERR_HIP, "conv_pgemm: %llu bytes of LDS refused", (unsigned long long)lds);
    }
    const dim3 grid(rpi * batch * mtiles);
    void* kargs[] = {&g};
    const hipError_t e = hipLaunchKernel(k, grid, dim3(kPgThreads), kargs, (size_t)lds, lc.s);
    if (e != hipSuccess) return cm_set_error(CM_ERR_HIP, "conv_pgemm: %s", hipGetErrorString(e));
    return cm_check_launch("conv_pgemm");
}

const int16_t* probe_ptr() {   // a 16-byte aligned stand-in for shape-only queries
    alignas(16) static const int16_t probe[8] = {};
    return probe;
}

}  // namespace

int cm_conv_pgemm_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                         uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                         uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                         uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                         uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc) {
    return pg_launch(x, w, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, sh, sw, dh,
                     dw, pad_top, pad_left, epi, lc, kPackAndRun, nullptr, nullptr, 0);
}

size_t cm_conv_pgemm_packed_bytes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                                  uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                                  uint32_t kw, uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
                                  uint32_t pad_top, uint32_t pad_left) {
    size_t need = 0;
    const LaunchCtx lc{nullptr, nullptr, 0, &need};
    const int16_t* p = probe_ptr();
    const int rc = pg_launch(p, p, p, const_cast<int16_t*>(p), batch, in_ch, in_h, in_w, out_ch, out_h,
                             out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left, nullptr, lc, kPackOnly,
                             nullptr, nullptr, 0);
    return rc == CM_OK ? need : 0u;
}

int cm_conv_pgemm_pack(const int16_t* w, uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                       uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                       uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                       uint32_t pad_left, void* dst, size_t bytes, hipStream_t s) {
    const LaunchCtx lc{s, nullptr, 0, nullptr};
    const int16_t* p = probe_ptr();
    const int rc = pg_launch(p, w, nullptr, const_cast<int16_t*>(p), batch, in_ch, in_h, in_w, out_ch,
                             out_h, out_w, kh, kw, sh, sw, dh, dw, pad_top, pad_left, nullptr, lc,
                             kPackOnly, nullptr, dst, bytes);
    return rc == 1 ? cm_set_error(CM_ERR_INVALID, "conv pack: the shape does not take the patch-GEMM path")
                   : rc;
}

int cm_conv_pgemm_run_packed(const int16_t* x, const void* packed, const int16_t* bias, int16_t* y,
                             uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                             uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                             uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                             uint32_t pad_left, const cm_epilogue_t* epi, hipStream_t s) {
    const LaunchCtx lc{s, nullptr, 0, nullptr};
    const int rc = pg_launch(x, nullptr, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                             sh, sw, dh, dw, pad_top, pad_left, epi, lc, kRunPacked, packed, nullptr, 0);
    return rc == 1 ? cm_set_error(CM_ERR_INVALID, "conv packed: the shape does not take the patch-GEMM path")
                   : rc;
}

// ------------------------------------------------------------- conv pair --
// A standard convolution (the patch GEMM, every middle channel in one row tile)
// with act1 applied, then a 1x1 convolution of its output, in one launch.
size_t cm_conv_pair_pgemm_bytes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                                 uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                                 uint32_t kw, uint32_t stride, uint32_t dilation, uint32_t pad_top,
                                 uint32_t pad_left, uint32_t out_ch) {
    size_t need = 0;
    const LaunchCtx lc{nullptr, nullptr, 0, &need};
    const int16_t* p = probe_ptr();
    const PairSpec ps{p, p, out_ch, 0u};
    const int rc = pg_launch(p, p, p, const_cast<int16_t*>(p), batch, in_ch, in_h, in_w, mid_ch, out_h,
                             out_w, kh, kw, stride, stride, dilation, dilation, pad_top, pad_left, nullptr,
                             lc, kPackOnly, nullptr, nullptr, 0, &ps);
    return rc == CM_OK ? need : 0u;
}

int cm_conv_pair_pgemm_pack(const int16_t* w1, const int16_t* w2, uint32_t batch, uint32_t in_ch, uint32_t in_h,
                      uint32_t in_w, uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                      uint32_t kw, uint32_t stride, uint32_t dilation, uint32_t pad_top, uint32_t pad_left,
                      uint32_t out_ch, void* dst, size_t bytes, hipStream_t s) {
    const LaunchCtx lc{s, nullptr, 0, nullptr};
    const int16_t* p = probe_ptr();
    const PairSpec ps{w2, nullptr, out_ch, 0u};
    const int rc = pg_launch(p, w1, nullptr, const_cast<int16_t*>(p), batch, in_ch, in_h, in_w, mid_ch,
                             out_h, out_w, kh, kw, stride, stride, dilation, dilation, pad_top, pad_left,
                             nullptr, lc, kPackOnly, nullptr, dst, bytes, &ps);
    return rc == 1 ? cm_set_error(CM_ERR_INVALID, "conv pair pack: the shapes do not take the pair path") : rc;
}

int cm_conv_pair_pgemm_run(const int16_t* x, const void* packed, const int16_t* bias1, const int16_t* bias2,
                            int16_t* y, uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                            uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                            uint32_t stride, uint32_t dilation, uint32_t pad_top, uint32_t pad_left,
                            uint32_t out_ch, uint32_t act1, const cm_epilogue_t* epi2, hipStream_t s) {
    const LaunchCtx lc{s, nullptr, 0, nullptr};
    const PairSpec ps{nullptr, bias2, out_ch, act1};
    const int rc = pg_launch(x, nullptr, bias1, y, batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw,
                             stride, stride, dilation, dilation, pad_top, pad_left, epi2, lc, kRunPacked,
                             packed, nullptr, 0, &ps);
    return rc == 1 ? cm_set_error(CM_ERR_INVALID, "conv pair: the shapes do not take the pair path") : rc;
}
