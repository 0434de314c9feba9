// gemm_dma.hip -- large dense Q8.8 MatMul on int8 MFMA with operands streamed
// into LDS by the memory system (direct-to-LDS buffer loads), four k steps deep.
//
// Reference arithmetic (kernels/matmul/kernel/MatmulKernel.cpp:196-218):
//     C[bi] = sat16( wrap32( A[bi] x B[bi] ) >> 8 ),  int16 A [n][k], B [k][m].
//
// Limbs as in gemm.hip: v = 256*vh + vl + 128 with vh = v >> 8 and
// vl = (v & 255) - 128, both int8, so that
//     sum a*b = 65536*S_hh + 256*S_mid + S_ll + 128*(sum_k a + sum_k b) - 16384*Kp
// over Kp = 64 * steps positions (zero padding adds 0 to both sides), every term
// mod 2^32 -- the ap_fixed<32,16> accumulator's wrap.  |S_mid| < 2^15 * K, so K
// is at most 32768 here (no fold).
//
// Two launches:
//   gemm_bpack  splits B once per call into MFMA-ready limb fragments in the
//               caller's workspace: for k step s (64 k) and 16-column tile t,
//               two 1 KB fragments (high, low limb) in which lane l's 16 bytes
//               are column 16t + (l % 16), k = 64s + 16(l / 16) + 0..15 -- the
//               B operand of v_mfma_i32_16x16x64_i8 -- and the column sums;
//               a 64 x 128 tile goes through LDS so that global reads are
//               16-byte rows and writes whole fragments;
//   gemm_dma    one block per 128 x 128 output tile: per k step the raw A tile
//               (128 rows x 64 k int16, 16 KB) and the tile's eight B fragment
//               pairs (16 KB) are loaded by buffer_load ... lds straight into one
//               of four LDS stages -- no registers and no ALU work, so three
//               steps are in flight while one is computed.  Eight waves hold
//               32 x 64 outputs each (2 x 4 MFMA tiles, three accumulator sets);
//               a wave reads its A fragments as raw int16 (a row's 16 k values,
//               two 16-byte reads) and splits them in registers (eight v_perm,
//               the row sums with v_dot2), its B fragments as they are.
//
// A's LDS rows are 128 bytes; the 16-byte chunk c of row r sits at position
// c ^ ((r >> 1) & 7), so the 16 rows of one fragment read fall in 16 distinct
// 16-byte bank groups.  The direct-to-LDS load writes lane i's 16 bytes at slot
// i of its 1 KB, so the swizzle is applied by choosing which chunk lane i loads.
#include "cm_internal.h"
#include "q88.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef short v2s __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kThreads = 512;
constexpr uint32_t BM = 128, BN = 128, BK = 64;
constexpr uint32_t kStages = 4;
constexpr uint32_t kStageA = BM * BK * 2;          // 16 KB raw int16
constexpr uint32_t kStageB = (BN / 16) * 2048;     // 8 fragment pairs, 16 KB
constexpr uint32_t kStage = kStageA + kStageB;
constexpr uint32_t kTilePitch = 132;               // epilogue tile row pitch (words)
constexpr uint32_t kMaxK = 32768;
constexpr uint32_t kGroupRows = 8;                 // row tiles per group of the tile order
constexpr uint64_t kPackBlocks = 1024;             // pack grid target (four per CU of an MI355X)

struct DmaArgs {
    const int16_t* a;
    const uint8_t* bp;       // packed B fragments
    const uint32_t* bsum;    // column sums of B, per packed batch
    int16_t* c;
    uint32_t n, k, m;
    uint32_t nk, nct8;       // k steps; column tiles per packed batch (multiple of 8)
    uint32_t nkc;            // k chunks of the pack: partial column sums per column
    uint32_t tiles_x, tiles_y, ntiles;   // column / row tiles; per batch
    uint64_t a_bs, c_bs;     // elements
    uint64_t bp_bs, bsum_bs; // bytes / words per packed batch (0: broadcast)
    EpiArgs epi;
};

struct PackArgs {
    const int16_t* b;
    uint8_t* bp;
    uint32_t* bsum;          // [packed batch][k chunk][nct8 * 16] partial column sums
    uint32_t k, m, nk, nct8;
    uint32_t spc;            // k steps per chunk (blockIdx.z: the chunk)
    uint64_t b_bs;           // elements between batches of B
    uint64_t bp_bs, bsum_bs;
};

__device__ __forceinline__ uint32_t hi4(uint32_t w0, uint32_t w1) {
    return __builtin_amdgcn_perm(w1, w0, 0x07050301u);
}
__device__ __forceinline__ uint32_t lo4(uint32_t w0, uint32_t w1) {
    return __builtin_amdgcn_perm(w1, w0, 0x06040200u) ^ 0x80808080u;
}
__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// ------------------------------------------------------------------ pack --
// Block (group of eight 16-column tiles, packed batch); four waves, each owning
// two of the eight tiles for every k step.  Per step the 64 x 128 int16 tile is
// read with 16-byte loads (rows past K and columns past M read 0), stored to LDS
// at a 260-byte row pitch, and each lane gathers its column's 16 k values.
constexpr uint32_t kPackPitch = 260;   // bytes: the four k groups of a gather hit distinct banks

__global__ __launch_bounds__(256) void gemm_bpack(PackArgs p) {
    __shared__ __align__(16) uint8_t t[BK * kPackPitch];
    touch_lines(p);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t grp = blockIdx.x, bb = blockIdx.y, kc = blockIdx.z;
    const uint32_t s_lo = kc * p.spc, s_hi = min(s_lo + p.spc, p.nk);
    const uint32_t c0 = grp * 128u;
    const int16_t* bbase = p.b + (uint64_t)bb * p.b_bs;
    const uint32_t cols_left = p.m > c0 ? p.m - c0 : 0u;
    uint8_t* out = p.bp + (uint64_t)bb * p.bp_bs;
    int32_t csum[2] = {0, 0};
    for (uint32_t s = s_lo; s < s_hi; ++s) {
        const uint32_t k0 = s * BK;
        const uint32_t krows = p.k - k0 < BK ? p.k - k0 : BK;
        // rows [k0, k0 + krows) of columns [c0, c0 + cols_left), 16-byte chunks
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(bbase + (uint64_t)k0 * p.m + c0,
                                                    ((krows - 1) * p.m + (cols_left < 128u ? cols_left : 128u)) * 2u);
        v4u d[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t u = q * 256u + tid, row = u >> 4, ch = u & 15u;
            const bool ok = row < krows && ch * 8u < cols_left;
            d[q] = __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? (row * p.m + ch * 8u) * 2u : kOob, 0, 0);
        }
        __syncthreads();   // the previous step's gathers are done
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t u = q * 256u + tid, row = u >> 4, ch = u & 15u;
            uint32_t* dst = reinterpret_cast<uint32_t*>(t + row * kPackPitch + ch * 16u);
            dst[0] = d[q][0]; dst[1] = d[q][1]; dst[2] = d[q][2]; dst[3] = d[q][3];
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t ct = wave * 2u + h;                 // tile within the group
            const uint32_t col = ct * 16u + (lane & 15u);
            const uint32_t kg = lane >> 4;
            uint32_t v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e)
                v[e] = *reinterpret_cast<const uint16_t*>(t + (kg * 16u + e) * kPackPitch + col * 2u);
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t w0 = pack2(v[4 * q], v[4 * q + 1]), w1 = pack2(v[4 * q + 2], v[4 * q + 3]);
                hw[q] = hi4(w0, w1);
                lw[q] = lo4(w0, w1);
                csum[h] += (int32_t)(int16_t)v[4 * q] + (int32_t)(int16_t)v[4 * q + 1] +
                           (int32_t)(int16_t)v[4 * q + 2] + (int32_t)(int16_t)v[4 * q + 3];
            }
            uint8_t* f = out + ((uint64_t)s * p.nct8 + grp * 8u + ct) * 2048u + lane * 16u;
            *reinterpret_cast<v4u*>(f) = v4u{hw[0], hw[1], hw[2], hw[3]};
            *reinterpret_cast<v4u*>(f + 1024) = v4u{lw[0], lw[1], lw[2], lw[3]};
        }
    }
    // column sums: the four k groups of a column are lanes l, l+16, l+32, l+48
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        int32_t v = csum[h];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        if (lane < 16u)
            p.bsum[(uint64_t)bb * p.bsum_bs + (uint64_t)kc * p.nct8 * 16u + c0 + (wave * 2u + h) * 16u + lane] =
                (uint32_t)v;
    }
}

// ------------------------------------------------------------------ main --
// A raw buffer descriptor in scalar registers (the same words make_rsrc builds:
// base, num_records bytes, 32-bit data, loads past the range read 0).
__device__ __forceinline__ v4u sdesc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return v4u{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a),
               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xFFFFu),
               (uint32_t)__builtin_amdgcn_readfirstlane(bytes), (uint32_t)kBufferWord3};
}
// One stage of loads: 16 bytes per lane from buffer da at byte offsets a0, a1
// into LDS at la0 / la1 + lane * 16, then the same from buffer db at b0, b1 into
// lb0 / lb1 (each LDS address goes through M0). Issued as inline asm: the
// compiler then neither waits for these loads before every LDS read (it cannot
// tell the stages apart) nor counts them; the kernel waits for them itself
// (wait_vm before the barrier that publishes a stage). M0 is saved first and
// restored last, so the asm leaves it as it found it.
__device__ __forceinline__ void dma_stage(const v4u& da, uint32_t a0, uint32_t a1, uint32_t la0, uint32_t la1,
                                          const v4u& db, uint32_t b0, uint32_t b1, uint32_t lb0, uint32_t lb1) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %5, %9, 0 offen lds\n\t"
                 "s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %6, %9, 0 offen lds\n\t"
                 "s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %7, %10, 0 offen lds\n\t"
                 "s_mov_b32 m0, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %8, %10, 0 offen lds\n\t"
                 "s_nop 0\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(__builtin_amdgcn_readfirstlane(la0)), "s"(__builtin_amdgcn_readfirstlane(la1)),
                   "s"(__builtin_amdgcn_readfirstlane(lb0)), "s"(__builtin_amdgcn_readfirstlane(lb1)),
                   "v"(a0), "v"(a1), "v"(b0), "v"(b1), "s"(da), "s"(db)
                 : "memory");
}

template <uint32_t N>
__device__ __forceinline__ void wait_vm() {
    // vmcnt(N) alone: expcnt / lgkmcnt fields at their maxima (no wait)
    static_assert(N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((int)((N & 15u) | ((N >> 4) << 14) | (0x7u << 4) | (0xFu << 8)));
}

__global__ __launch_bounds__(kThreads, 1) void gemm_dma(DmaArgs g) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t row_sum[BM];
    __shared__ uint32_t col_sum[BN];
    touch_lines(g);
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    // XCD-aware order: workgroups are dealt to the 8 XCDs round robin; XCD x
    // takes the x-th contiguous share of the (batch, row tile, column tile)
    // order, so that blocks sharing A rows and B columns meet in one L2
    const uint32_t nb = gridDim.x, per = nb >> 3, rem = nb & 7u, xcd = blockIdx.x & 7u, idx = blockIdx.x >> 3;
    const uint32_t lg = xcd < rem ? xcd * (per + 1u) + idx : rem * (per + 1u) + (xcd - rem) * per + idx;
    // within a batch, tiles go in groups of kGroupRows row tiles, column by column,
    // so the blocks that run together on one XCD share few A and B panels
    const uint32_t bz = lg / g.ntiles, tt = lg - bz * g.ntiles;
    const uint32_t gsize = kGroupRows * g.tiles_x, grp = tt / gsize;
    const uint32_t first = grp * kGroupRows;
    const uint32_t rows_in = min(g.tiles_y - first, kGroupRows);
    const uint32_t in_grp = tt - grp * gsize;
    const uint32_t by = first + in_grp % rows_in, bx = in_grp / rows_in;
    const uint32_t row0 = by * BM, col0 = bx * BN;
    const uint32_t wr = wave & 3u, wc = wave >> 2;     // wave rows 32 * wr, columns 64 * wc

    // A: the block's rows of batch bz; rows past n read 0 through the range
    const uint32_t arows = g.n - row0 < BM ? g.n - row0 : BM;
    const v4u ars = sdesc(g.a + (uint64_t)bz * g.a_bs + (uint64_t)row0 * g.k, arows * g.k * 2u);
    // B fragments of batch bz (the packed region's step s starts at s * nct8 * 2 KB)
    const v4u brs = sdesc(g.bp + (uint64_t)bz * g.bp_bs, g.nk * g.nct8 * 2048u);
    const uint32_t lds0 = (uint32_t)reinterpret_cast<uintptr_t>((lds_void*)lds);

    // this thread's two A chunks (slots u = q * 512 + tid of the 1024) and two B chunks
    uint32_t a_off[2], a_kc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t u = q * kThreads + tid, row = u >> 3, pos = u & 7u;
        const uint32_t c = pos ^ ((row >> 1) & 7u);   // logical chunk that lands at this slot
        a_kc[q] = c * 8u;
        a_off[q] = (row * g.k + c * 8u) * 2u;
    }
    auto issue = [&](uint32_t s) {
        const uint32_t st = lds0 + (s % kStages) * kStage + wave * 64u * 16u;
        const uint32_t k0 = s * BK;
        // A chunks at or past K (and every chunk of a step past the last) read 0
        const uint32_t a0 = k0 + a_kc[0] < g.k ? a_off[0] + k0 * 2u : kOob;
        const uint32_t a1 = k0 + a_kc[1] < g.k ? a_off[1] + k0 * 2u : kOob;
        const uint32_t bbase = s < g.nk ? (s * g.nct8 + bx * 8u) * 2048u : kOob;
        const uint32_t b0 = bbase == kOob ? kOob : bbase + tid * 16u;
        const uint32_t b1 = bbase == kOob ? kOob : bbase + (kThreads + tid) * 16u;
        dma_stage(ars, a0, a1, st, st + kThreads * 16u,
                  brs, b0, b1, st + kStageA, st + kStageA + kThreads * 16u);
    };

    v4i hh[2][4], mid[2][4], ll[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) hh[i][j] = mid[i][j] = ll[i][j] = v4i{0, 0, 0, 0};
    // A row sums: the two waves of a wave row read the same 32 A rows, so each
    // sums 16 of them: wave column wc holds row tile wc as its fragment set 0
    // (set i is row tile i ^ wc) and sums set 0's words
    int32_t rsum = 0;

    // fragment addresses: A row r = 32 wr + 16 i + (lane % 16), logical chunks 2q, 2q + 1
    const uint32_t q4 = lane >> 4;
    uint32_t a_rd[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t r = wr * 32u + (i ^ wc) * 16u + (lane & 15u), f = (r >> 1) & 7u;
        a_rd[i][0] = r * 128u + (((2u * q4) ^ f) << 4);
        a_rd[i][1] = r * 128u + (((2u * q4 + 1u) ^ f) << 4);
    }
    const uint32_t b_rd = kStageA + wc * 4u * 2048u + lane * 16u;

    // Fragments of one k step: read from LDS one step ahead, so that a step's
    // MFMAs start right after the barrier while the next step's reads are in flight.
    struct Frags {
        v4i bh[4], bl[4];
        v4u r0[2], r1[2];
    };
    auto read_frags = [&](uint32_t s, Frags& f) {
        const uint8_t* st = lds + (s % kStages) * kStage;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f.bh[j] = *reinterpret_cast<const v4i*>(st + b_rd + j * 2048u);
            f.bl[j] = *reinterpret_cast<const v4i*>(st + b_rd + j * 2048u + 1024u);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            f.r0[i] = *reinterpret_cast<const v4u*>(st + a_rd[i][0]);
            f.r1[i] = *reinterpret_cast<const v4u*>(st + a_rd[i][1]);
        }
    };
    auto row_words = [&](const v4u& r0, const v4u& r1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // (a vector element copied out first: bit_cast of r0[e] itself reads r0[0])
            const uint32_t w0 = r0[e], w1 = r1[e];
            rsum = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, w0), v2s{1, 1}, rsum, false);
            rsum = __builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, w1), v2s{1, 1}, rsum, false);
        }
    };
    auto compute = [&](const Frags& f) {
        row_words(f.r0[0], f.r1[0]);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const v4u r0 = f.r0[i], r1 = f.r1[i];
            const v4i ah = v4i{(int)hi4(r0[0], r0[1]), (int)hi4(r0[2], r0[3]),
                               (int)hi4(r1[0], r1[1]), (int)hi4(r1[2], r1[3])};
            const v4i al = v4i{(int)lo4(r0[0], r0[1]), (int)lo4(r0[2], r0[3]),
                               (int)lo4(r1[0], r1[1]), (int)lo4(r1[2], r1[3])};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                hh[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, f.bh[j], hh[i][j], 0, 0, 0);
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah, f.bl[j], mid[i][j], 0, 0, 0);
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, f.bh[j], mid[i][j], 0, 0, 0);
                ll[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al, f.bl[j], ll[i][j], 0, 0, 0);
            }
        }
    };

    // Pipeline: all four stages loading at first; iteration s waits until step
    // s + 1 has landed (three steps were in flight), and after the barrier --
    // every wave has read step s's stage into registers -- loads step s + 4
    // into that stage, reads step s + 1's fragments and computes step s.
#pragma unroll
    for (uint32_t s = 0; s < kStages; ++s) issue(s);
    wait_vm<(kStages - 1) * 4>();   // step 0
    __syncthreads();
    Frags fa, fb;
    read_frags(0, fa);
    for (uint32_t s = 0; s < g.nk; s += 2) {
        wait_vm<(kStages - 2) * 4>();   // step s + 1 (past the last: zeros)
        __syncthreads();
        issue(s + kStages);
        read_frags(s + 1, fb);
        compute(fa);
        if (s + 1 >= g.nk) break;
        wait_vm<(kStages - 2) * 4>();
        __syncthreads();
        issue(s + 1 + kStages);
        read_frags(s + 2, fa);
        compute(fb);
    }
    wait_vm<0>();        // the (empty) loads past the last step
    __syncthreads();     // every wave is done with the stages: the tile may reuse them

    // row sums (lanes l, l+16, l+32, l+48 hold one row's four k groups) and column sums
    {
        int32_t v = rsum;
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        if (lane < 16u) row_sum[wr * 32u + wc * 16u + lane] = (uint32_t)v;
    }
    if (tid < BN) {
        const uint32_t c = col0 + tid;
        uint32_t v = 0;
        const uint32_t* bs = g.bsum + (uint64_t)bz * g.bsum_bs + c;
        for (uint32_t kc = 0; kc < g.nkc; ++kc) v += bs[(uint64_t)kc * g.nct8 * 16u];
        col_sum[tid] = c < g.m ? v : 0u;
    }
    uint32_t* tile = reinterpret_cast<uint32_t*>(lds);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t v = ((uint32_t)hh[i][j][e] << 16) + ((uint32_t)mid[i][j][e] << 8) +
                                   (uint32_t)ll[i][j][e];
                tile[(wr * 32u + (i ^ wc) * 16u + q4 * 4u + e) * kTilePitch + wc * 64u + j * 16u + (lane & 15u)] = v;
            }
    __syncthreads();

    // row-major: thread t finishes columns [c8, c8 + 8) of rows rb, rb + 32, rb + 64, rb + 96
    const uint32_t c8 = (tid & 15u) * 8u, rb = tid >> 4;
    const uint32_t cbase = col0 + c8;
    if (cbase >= g.m) return;   // m % 8 == 0: a group of 8 columns is all in or all out
    const uint32_t kp_term = 16384u * (g.nk * BK);
    uint32_t cterm[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) cterm[q] = 128u * col_sum[c8 + q] - kp_term;
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    int32_t cadd[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (g.epi.add_mode == 2u) {
#pragma unroll
        for (int q = 0; q < 8; ++q) cadd[q] = g.epi.add[cbase + q];
    }
    int16_t* cp = g.c + (uint64_t)bz * g.c_bs;
    const int16_t* ap = g.epi.add + (uint64_t)bz * g.c_bs;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const uint32_t r = rb + rr * 32u;
        if (row0 + r >= g.n) break;
        const uint64_t o = (uint64_t)(row0 + r) * g.m + cbase;
        const v4u t0 = *reinterpret_cast<const v4u*>(&tile[r * kTilePitch + c8]);
        const v4u t1 = *reinterpret_cast<const v4u*>(&tile[r * kTilePitch + c8 + 4]);
        const uint32_t rs = 128u * row_sum[r];
        int32_t add[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) add[q] = cadd[q];
        if (g.epi.add_mode == 1u) {
            const v4u v = *reinterpret_cast<const v4u*>(ap + o);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                add[2 * q] = (int32_t)(int16_t)(v[q] & 0xFFFFu);
                add[2 * q + 1] = (int32_t)v[q] >> 16;
            }
        }
        int32_t y[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t v = (q < 4 ? t0[q] : t1[q - 4]) + cterm[q] + rs;
            int32_t d = q88::acc_to_data(v);
            if (g.epi.add_mode) d = q88::add(d, add[q]);
            y[q] = q88::clamp(d, lo, hi);
        }
        *reinterpret_cast<v4u*>(cp + o) = v4u{pack2((uint32_t)y[0] & 0xFFFFu, (uint32_t)y[1] & 0xFFFFu),
                                              pack2((uint32_t)y[2] & 0xFFFFu, (uint32_t)y[3] & 0xFFFFu),
                                              pack2((uint32_t)y[4] & 0xFFFFu, (uint32_t)y[5] & 0xFFFFu),
                                              pack2((uint32_t)y[6] & 0xFFFFu, (uint32_t)y[7] & 0xFFFFu)};
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// Dense batched MatMul on the direct-to-LDS path, or 1 when the call does not
// take it (the caller runs the general GEMM).  The packed B goes to the caller's
// workspace; with lc.need set the bytes it would use are reported and 1 is
// returned, so that the general path adds its own (split-K) need.
int cm_gemm_dma_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                       uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs,
                       const cm_epilogue_t* epi, const LaunchCtx& lc) {
    if (batch == 0 || n == 0 || m == 0) return 1;
    // large products only (enough 128 x 128 tiles to fill the chip), 16-byte rows
    // and batch steps everywhere, and outputs of different batches disjoint
    const uint64_t tiles = (uint64_t)batch * ((n + BM - 1) / BM) * ((m + BN - 1) / BN);
    const bool shape = tiles >= 256 && k >= 256 && k <= kMaxK && k % 8 == 0 && m % 8 == 0 &&
                       a_bs % 8 == 0 && b_bs % 8 == 0 && c_bs % 8 == 0 &&
                       (batch == 1 || (uint64_t)c_bs >= (uint64_t)n * m) && tiles < (1ull << 31) &&
                       (uint64_t)n * k * 2 < (1ull << 31) && (uint64_t)k * m * 2 < (1ull << 31);
    if (!shape || !aligned16(a) || !aligned16(b) || !aligned16(c)) return 1;
    const EpiArgs ep = cm_epi_args(epi);
    if (ep.add_mode == 1u && (!aligned16(ep.add) || ep.add == nullptr)) return 1;
    if (ep.add_mode > 2u || (ep.add_mode && ep.add == nullptr)) return 1;
    const uint32_t nk = (k + BK - 1) / BK;
    const uint32_t nct8 = (m + 127u) / 128u * 8u;
    const uint32_t nbb = b_bs == 0 ? 1u : batch;   // B broadcast over the batch: packed once
    if (nbb > 65535u) return 1;                     // the pack grid's y extent
    // pack grid: column groups x packed batches x k chunks, about kPackBlocks
    // blocks (a fixed target, so that the workspace size depends on the shape only)
    const uint64_t pack_blocks = (uint64_t)(nct8 / 8u) * nbb;
    const uint64_t want_kc = (kPackBlocks + pack_blocks - 1) / pack_blocks;
    const uint32_t spc = (uint32_t)((nk + (want_kc < nk ? want_kc : nk) - 1) / (want_kc < nk ? want_kc : nk));
    const uint32_t nkc = (nk + spc - 1) / spc;
    const uint64_t bp_bs = (uint64_t)nk * nct8 * 2048u;
    const uint64_t bsum_bs = (uint64_t)nkc * nct8 * 16u;
    if (bp_bs >= (1ull << 31)) return 1;
    const uint64_t need = nbb * bp_bs + nbb * bsum_bs * 4u;
    if (lc.need) {   // size query: report this path's bytes, let the general path add its own
        if (need > *lc.need) *lc.need = need;
        return 1;
    }
    if (!lc.ws || lc.ws_bytes < need || !aligned16(lc.ws)) return 1;
    uint8_t* bp = static_cast<uint8_t*>(lc.ws);
    uint32_t* bsum = reinterpret_cast<uint32_t*>(bp + nbb * bp_bs);

    PackArgs pa{b, bp, bsum, k, m, nk, nct8, spc, b_bs, bp_bs, bsum_bs};
    hipLaunchKernelGGL(gemm_bpack, dim3(nct8 / 8u, nbb, nkc), dim3(256), 0, lc.s, pa);
    int rc = cm_check_launch("gemm_bpack");
    if (rc) return rc;

    DmaArgs g{};
    g.a = a; g.bp = bp; g.bsum = bsum; g.c = c;
    g.n = n; g.k = k; g.m = m; g.nk = nk; g.nct8 = nct8; g.nkc = nkc;
    g.tiles_x = (m + BN - 1) / BN; g.tiles_y = (n + BM - 1) / BM;
    g.ntiles = g.tiles_x * g.tiles_y;
    g.a_bs = a_bs; g.c_bs = c_bs;
    g.bp_bs = b_bs == 0 ? 0u : bp_bs;
    g.bsum_bs = b_bs == 0 ? 0u : bsum_bs;
    g.epi = ep;
    static bool attr_set[64] = {};
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev >= 0 && dev < 64 && !attr_set[dev]) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kStages * kStage) != hipSuccess)
            return cm_set_error(CM_ERR_HIP, "gemm_dma: cannot set the LDS size");
        attr_set[dev] = true;
    }
    hipLaunchKernelGGL(gemm_dma, dim3((uint32_t)tiles), dim3(kThreads), kStages * kStage, lc.s, g);
    return cm_check_launch("gemm_dma");
}
