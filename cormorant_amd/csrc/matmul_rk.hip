// matmul_rk.hip -- small matrix products on int8 MFMA with the operands loaded
// straight into registers (kernels/matmul/kernel/MatmulKernel.cpp:196-218).
//
// C[n][m] = sat16(wrap32(sum_k A[n][k] * B[k][m]) >> 8), then the optional fused
// epilogue (Add of a same-shaped tensor or of a row vector per column, then
// Relu / Relu6).  One product, batch 1.
//
// A network's classifier layers (an MLP's 64 x 784 x 256, a 16 x 1280 x 1000
// head) have a few dozen 128 x 128 tiles at most, so the block-tiled GEMM walks
// K serially in a handful of blocks or splits it over blocks and adds a reduce
// launch.  Here a block of four waves (eight from eight k steps on) owns one
// 32 x 32 output tile and splits the reduction over its waves (wave w of NW
// takes k steps w, w + NW, ...); each wave
// loads its MFMA fragments straight into registers -- A, 16 consecutive k of
// one row, with 16-byte loads when rows allow; B, 16 k rows of one column,
// with 2-byte loads -- one k step ahead, splits the limbs in registers, and
// turns its accumulators into its partial sum of each output (mod 2^32).  The
// partials meet in LDS after one barrier and each wave finishes 1/NW of the
// tile.  An element outside the matrices gets bit 31 set in its buffer
// offset and reads 0 (a select on a validity flag became a branch per load).
//
// Limbs and the exact sum are the GEMM kernel's: v = 256*vh + vl + 128 with
// vh = v >> 8, vl = (v & 255) - 128, and over the k positions a wave processes
//     sum a*b = 65536*S_hh + 256*S_mid + S_ll + 128*(sum a + sum b) - 16384*Kp
// (a zero position contributes 0 to both sides), so the partials add up,
// modulo 2^32, to the whole reduction: the accumulator's own wrap.
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

constexpr uint32_t kMrMaxSteps = 64;      // k steps of 64 (at most 16 per wave)
constexpr uint64_t kMrMaxOut = 1u << 18;  // outputs: larger products fill the chip with the GEMM

struct MrArgs {
    const int16_t* a;
    const int16_t* b;
    int16_t* c;
    EpiArgs epi;
    uint32_t n, k, m;
    uint32_t lda, ldc;          // elements between rows of A and of C (and of a same-shaped Add)
    uint32_t rt, nk;            // row tiles of 32, k steps of 64
    uint32_t a_bytes, b_bytes, c_bytes;
};

struct MrStep {
    uint32_t a[2][8];    // two rows, 16 k as packed words
    uint32_t b[2][16];   // two columns, 16 k, one int16 per register
};

template <bool AV>
__device__ __forceinline__ void mr_load(const MrArgs& g, __amdgpu_buffer_rsrc_t ar, __amdgpu_buffer_rsrc_t br,
                                        const uint32_t (&arow)[2], const uint32_t (&bcol)[2], uint32_t k0,
                                        MrStep& st) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (AV) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                // k % 8 == 0: a group of 8 k values is wholly inside or outside the
                // row; an invalid row's arow is kOob, a k past the end sets bit 31
                const uint32_t hole = (uint32_t)(k0 + q * 8 >= g.k) << 31;
                const v4u v = __builtin_amdgcn_raw_buffer_load_b128(ar, (arow[i] + (k0 + q * 8) * 2u) | hole, 0, 0);
                st.a[i][4 * q + 0] = v[0]; st.a[i][4 * q + 1] = v[1];
                st.a[i][4 * q + 2] = v[2]; st.a[i][4 * q + 3] = v[3];
            }
        } else {
            uint32_t r[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t hole = (uint32_t)(k0 + e >= g.k) << 31;
                r[e] = __builtin_amdgcn_raw_buffer_load_b16(ar, (arow[i] + (k0 + e) * 2u) | hole, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) st.a[i][e] = pack2(r[2 * e], r[2 * e + 1]);
        }
    }
    const uint32_t rst = g.m * 2u;   // bytes between two k rows of B
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            // an invalid column's bcol is kOob (the sum stays below 2^32)
            const uint32_t hole = (uint32_t)(k0 + e >= g.k) << 31;
            st.b[j][e] = __builtin_amdgcn_raw_buffer_load_b16(br, (bcol[j] + (k0 + e) * rst) | hole, 0, 0);
        }
}

// NW waves per block (4, or 8 for 8 or more k steps): the k steps split NW ways.
template <bool AV, int NW>
__global__ __launch_bounds__(64 * NW) void matmul_rk(MrArgs g) {
    static_assert(NW == 4 || NW == 8, "four or eight waves");
    constexpr uint32_t U = 16u / NW;   // outputs of the lane's 16 each wave finishes
    __shared__ uint32_t red[NW][16][64];   // each wave's partial sums
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t rt = blockIdx.x % g.rt, ct = blockIdx.x / g.rt;   // scalar: blockIdx is uniform
    const uint32_t r16 = lane & 15, kg = lane >> 4;
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(g.a, g.a_bytes), br = make_rsrc(g.b, g.b_bytes);
    uint32_t arow[2], bcol[2], col[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t r = rt * 32u + i * 16u + r16;
        arow[i] = r < g.n ? r * g.lda * 2u : kOob;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        col[j] = ct * 32u + j * 16u + r16;
        bcol[j] = col[j] < g.m ? col[j] * 2u : kOob;
    }
    // this wave finishes outputs v = U * wave + u of the lane's 16 (v = 8 * i +
    // 2 * e + j: row tile i, row 4 * kg + e, column j); their fused-Add operands
    // load now, behind the k loop
    uint32_t fadd[U] = {};
    if (g.epi.add_mode != 0u) {
        const uint32_t ab = g.epi.add_mode == 1u ? g.c_bytes : g.m * 2u;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(g.epi.add, ab);
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t v = U * wave + u, i = v >> 3, e = (v >> 1) & 3u, j = v & 1u;
            const uint32_t r = rt * 32u + i * 16u + kg * 4u + e;
            const bool ok = r < g.n && col[j] < g.m;
            const uint32_t el = g.epi.add_mode == 1u ? r * g.ldc + col[j] : col[j];
            fadd[u] = __builtin_amdgcn_raw_buffer_load_b16(xr, ok ? el * 2u : kOob, 0, 0);
        }
    }

    v4i hh[2][2], mid[2][2], ll[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) hh[i][j] = mid[i][j] = ll[i][j] = v4i{0, 0, 0, 0};
    int32_t ahs[2] = {0, 0}, als[2] = {0, 0}, bhs[2] = {0, 0}, bls[2] = {0, 0};
    auto compute = [&](const MrStep& st) {
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
    // this wave's steps s = wave, wave + NW, ... (two register stages; past the
    // last step the loads read 0 through the offsets' bit 31 and are never used)
    const uint32_t kl = kg * 16u;
    uint32_t my = 0;
    MrStep s0, s1;
    mr_load<AV>(g, ar, br, arow, bcol, wave * 64u + kl, s0);
    for (uint32_t s = wave; s < g.nk; s += 2 * NW) {
        mr_load<AV>(g, ar, br, arow, bcol, (s + NW) * 64u + kl, s1);
        compute(s0);
        ++my;
        if (s + NW >= g.nk) break;
        mr_load<AV>(g, ar, br, arow, bcol, (s + 2 * NW) * 64u + kl, s0);
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
    for (uint32_t u = 0; u < U; ++u) {
        const uint32_t v = U * wave + u, i = v >> 3, e = (v >> 1) & 3u, j = v & 1u;
        const uint32_t r = rt * 32u + i * 16u + kg * 4u + e;
        uint32_t acc = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) acc += red[w][v][lane];
        if (r >= g.n || col[j] >= g.m) continue;
        int32_t o = q88::acc_to_data(acc);
        if (g.epi.add_mode != 0u) o = q88::add(o, (int16_t)fadd[u]);
        g.c[r * g.ldc + col[j]] = (int16_t)q88::clamp(o, lo, hi);
    }
}

}  // namespace

// Returns 1 when the shape is not for this path (the caller takes the block GEMM).
// Rows of A lie lda elements apart and rows of C (and of a same-shaped Add) ldc
// apart: a batch of single-row products whose B is shared is one product here.
int cm_matmul_rk_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k, uint32_t m,
                        uint32_t lda, uint32_t ldc, const cm_epilogue_t* epi, const LaunchCtx& lc) {
    const uint64_t out = (uint64_t)n * m;
    if (n == 0 || m == 0 || k == 0 || out > kMrMaxOut || (k + 63u) / 64u > kMrMaxSteps) return 1;
    if (lda < k || ldc < m) return 1;
    const uint64_t a_span = 2ull * ((uint64_t)(n - 1) * lda + k), c_span = 2ull * ((uint64_t)(n - 1) * ldc + m);
    if (a_span >= 0x80000000ull || 2ull * k * m >= 0x80000000ull || c_span >= 0x80000000ull) return 1;
    if (lc.need) return CM_OK;   // no workspace
    MrArgs g{};
    g.a = a; g.b = b; g.c = c; g.epi = cm_epi_args(epi);
    g.n = n; g.k = k; g.m = m;
    g.lda = lda; g.ldc = ldc;
    g.rt = (n + 31) / 32;
    g.nk = (k + 63) / 64;
    g.a_bytes = (uint32_t)a_span;
    g.b_bytes = (uint32_t)(2ull * k * m);
    g.c_bytes = (uint32_t)c_span;
    const dim3 grid((uint32_t)((uint64_t)g.rt * ((m + 31) / 32)));
    // eight waves when there are eight or more k steps: each walks half as many
    const bool av = k % 8 == 0 && lda % 8 == 0 && ((uintptr_t)a & 15u) == 0;
    if (g.nk >= 8) {
        if (av) hipLaunchKernelGGL((matmul_rk<true, 8>), grid, dim3(512), 0, lc.s, g);
        else hipLaunchKernelGGL((matmul_rk<false, 8>), grid, dim3(512), 0, lc.s, g);
    } else {
        if (av) hipLaunchKernelGGL((matmul_rk<true, 4>), grid, dim3(256), 0, lc.s, g);
        else hipLaunchKernelGGL((matmul_rk<false, 4>), grid, dim3(256), 0, lc.s, g);
    }
    return cm_check_launch("matmul_rk");
}
