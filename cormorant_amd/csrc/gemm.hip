// gemm.hip -- exact Q8.8 GEMM and implicit-GEMM convolution on gfx950 int8 MFMA.
//
// Reference arithmetic (kernels/matmul/kernel/MatmulKernel.cpp:196-218,
// kernels/conv/kernel/ConvKernel.cpp:160-169, 231-249, 333):
//     acc = wrap32( [bias << 8] + sum_k a_k * b_k ),   out = sat16(acc >> 8)
// with int16 operands and an ap_fixed<32,16> accumulator that wraps mod 2^32.
//
// Limb decomposition.  Every int16 v splits into a signed high byte and an
// offset low byte, both int8:
//     vh = v >> 8,   vl = (v & 255) - 128,   v = 256*vh + vl + 128.
// With A' = a - 128 = 256*ah + al and B' = b - 128 = 256*bh + bl,
//     sum a*b = 65536*S_hh + 256*S_mid + S_ll + 128*(sum_k a + sum_k b) - 16384*Kp
// where S_hh = sum ah*bh, S_mid = sum (ah*bl + al*bh), S_ll = sum al*bl are
// int8 x int8 -> int32 MFMA sums over the Kp (zero-padded) k positions, and
// the row sums of A / column sums of B are gathered while tiles are loaded.
// Every term is taken modulo 2^32, which is exactly the accumulator's wrap,
// so the result is bit-identical to the reference for any inputs.  |S_mid|
// grows by at most 2^15 per k, so MFMA partials are folded into a uint32
// total every 32768 k when K is larger than that (never overflow int32).
//
// Tiling: 512 threads = 8 waves (2 x 4), block tile 128 rows x 128 cols x 64 k,
// wave tile 64 x 32 = 4 x 2 MFMA 16x16x64 tiles with 3 accumulator sets (hh,
// mid, ll): 96 accumulator registers, so two waves share each SIMD and one
// wave's MFMAs run while the other waits on memory or does its limb split.
// Tiles are split into limbs while being stored to LDS (see Planes for the
// layouts and their bank conflicts).  The next tile's loads are issued before the MFMA phase; loads are
// unconditional (out-of-range elements are zeroed by the buffer range check
// or by a select), so all of a tile's loads are in flight at once.
#include <type_traits>

#include "cm_internal.h"
#include "q88.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 512;
constexpr int kChunk = BM * 16;      // A planes: LDS bytes of one 16-byte k chunk of all 128 rows
constexpr int kStride = 80;          // B planes: LDS bytes per column of 64 int8 (k) values
constexpr int kFoldIters = 512;      // fold MFMA partials every 512*64 = 32768 k
constexpr int TI = 4, TJ = 2;        // MFMA tiles per wave: 4 row tiles x 2 column tiles
constexpr uint32_t kTabMax = 2048;   // largest K of the table-driven convolution gather

struct GemmArgs {
    const int16_t* a;     // [rows][k], row stride lda (weights for conv)
    const int16_t* b;     // dense: [k][cols], row stride ldb; conv: x (NCHW)
    int16_t* c;           // dense: [rows][cols], row stride ldc; conv: y (NCHW)
    const int16_t* bias;  // [rows] or null
    uint32_t rows, cols, k;
    uint64_t lda, ldb, ldc;
    uint64_t a_bs, b_bs, c_bs;   // per blockIdx.z (dense only)
    uint32_t a_vec, b_vec;       // A: 16-byte row loads; B: 8-byte row loads
    // implicit GEMM: column = n*P + p, k = (c*kh + khi)*kw + kwi
    uint32_t C, H, W, OW, P, kh, kw, sh, sw, dh, dw, pt, pl;
    uint64_t x_img, y_img;
    FastDiv div_p, div_ow, div_kk, div_kw;   // divisions by P, OW, kh*kw, kw
    uint32_t x_bytes;            // table mode: size of the whole input tensor, < 2^31
    EpiArgs epi;                 // fused Add / Relu / Clip; add_mode 1 follows C's layout
    // output (and add tensor) accesses of `out_w` elements at a time keep their
    // alignment and stay inside one image: out_w divides ldc / c_bs (dense) or
    // P (conv) and both base pointers are aligned to 2*out_w bytes
    uint32_t out_w;
    // split-K: blockIdx.z selects k steps [z*split_steps, +split_steps) and the
    // block stores its partial sums (no bias) to ws[z][row][0..ws_ld); ws_ld is
    // cols rounded up to 8; 0 = no split
    uint32_t split_steps, ws_ld;
    uint32_t* ws;
};

// Limb bytes of four int16 values held in two words w0 = (v0 | v1 << 16),
// w1 = (v2 | v3 << 16): one v_perm_b32 gathers the high bytes (v >> 8) and one
// more the low bytes, which the xor offsets by -128.  Byte i of the result is
// value i, so k order is preserved.
__device__ __forceinline__ uint32_t hi4(uint32_t w0, uint32_t w1) {
    return __builtin_amdgcn_perm(w1, w0, 0x07050301u);
}
__device__ __forceinline__ uint32_t lo4(uint32_t w0, uint32_t w1) {
    return __builtin_amdgcn_perm(w1, w0, 0x06040200u) ^ 0x80808080u;
}
// Sum of the four signed bytes of w added to acc (v_dot4 with a ones vector).
__device__ __forceinline__ int32_t bsum(uint32_t w, int32_t acc) {
    return __builtin_amdgcn_sdot4((int)w, 0x01010101, acc, false);
}
// Two zero-extended int16 values -> one word (lo | hi << 16).
__device__ __forceinline__ uint32_t pack(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// One k step's limb planes.  Two of them alternate: the MFMA phase reads one
// while the next tile is split into the other.
// Limb planes of 128 rows (A) / columns (B) x 64 int8 k values.
// A is chunk-major: k chunk q (16 bytes) of row r at q * kChunk + (r ^ 2q) * 16.
// An MFMA fragment read (16 lanes: rows r0..r0+15 of one chunk) covers one
// contiguous 256-byte block, and the staging stores (thread t: row t / 4,
// chunk t % 4, so that a load quad reads one row) land in distinct banks: the
// XOR moves the four chunks of a row pair to eight different 16-byte slots.  B keeps one 80-byte row per column: its staging
// is 4-byte stores of 2 columns x 16 k words (paired into ds_write2, no
// conflict); its fragment reads conflict.  Measured on single-pattern LDS
// kernels with the bank-conflict counter: an 80-byte pitch costs 4 conflict
// cycles per fragment read and 8 per 16-byte store of 4 chunks x 4 rows; the
// chunk-major reads and stores cost none.  A chunk-major B (with an XOR of the
// column by the chunk against the stores' conflicts) removed the rest of the
// conflicts but ran 10 % slower: its addresses no longer pair into ds_write2
// or fold into immediate offsets.
struct Planes {
    uint8_t a_hi[4 * kChunk];
    uint8_t a_lo[4 * kChunk];
    uint8_t b_hi[BN * kStride];
    uint8_t b_lo[BN * kStride];
};
__device__ __forceinline__ uint32_t a_off(uint32_t r, uint32_t q) { return q * kChunk + ((r ^ (q << 1)) << 4); }

// A staging: thread t owns row a_row(t) and k chunk a_chunk(t); the four threads
// of a row are adjacent lanes, so each load quad reads one row's 128 bytes.
__device__ __forceinline__ uint32_t a_row(uint32_t t) { return t >> 2; }
__device__ __forceinline__ uint32_t a_chunk(uint32_t t) { return t & 3u; }

// Epilogue tile: the block's 128 x 128 raw sums, rows padded to 132 words so
// the four row groups of an MFMA result write fall into different bank halves.
constexpr int kTilePitch = 132;

struct Smem {
    union {
        Planes st[2];                        // main loop
        uint32_t tile[BM * kTilePitch];      // epilogue (after the last k step)
    };
    uint32_t row_sum[BM];
    uint32_t col_sum[BN];
    int32_t bias[BM];      // bias << 8 of the block's rows (0 past the last row)
    uint64_t coff[BN];     // convolution: output offset n*y_img + p of each column
};

// Splits 16 int16 values (8 packed words, k order) into 16 high and 16 low
// limb bytes, stores both at byte offset `off` of the two planes, and adds the
// limb sums to hs / ls.
__device__ __forceinline__ void store16(uint8_t* hi_plane, uint8_t* lo_plane, uint32_t off,
                                        const uint32_t (&w)[8], int32_t& hs, int32_t& ls) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hi[j] = hi4(w[2 * j], w[2 * j + 1]);
        lo[j] = lo4(w[2 * j], w[2 * j + 1]);
        hs = bsum(hi[j], hs);
        ls = bsum(lo[j], ls);
    }
    *reinterpret_cast<v4i*>(hi_plane + off) = v4i{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    *reinterpret_cast<v4i*>(lo_plane + off) = v4i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
}

// ---------------------------------------------------------------- A tile --
// Thread t owns row a_row(t) and k values [16 * a_chunk(t), +16) of the 64-k slice.  The
// loads only fill registers (8 words for 16-byte loads, 16 raw values
// otherwise); packing and the limb split happen in store(), after the MFMA
// phase, so every load of a tile is in flight at once.
struct ATile {
    uint32_t w[8];      // vector path: two int16 per word
    uint32_t raw[16];   // element path: one int16 per register

    // Global loads (any size): out-of-range elements read a valid address of
    // the same row and are zeroed afterwards.
    __device__ __forceinline__ void load(const GemmArgs& g, const int16_t* abase, uint32_t row0,
                                         uint32_t k0) {
        const uint32_t r = row0 + a_row(threadIdx.x);
        const uint32_t ks = k0 + a_chunk(threadIdx.x) * 16;
        const bool rok = r < g.rows;
        const int16_t* p = abase + (uint64_t)(rok ? r : 0u) * g.lda;
        if (g.a_vec) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const bool ok = rok && ks + q * 8 < g.k;
                v4i v = *reinterpret_cast<const v4i*>(p + (ok ? ks + q * 8 : 0u));
                const v4i z = {0, 0, 0, 0};
                v = ok ? v : z;
                w[4 * q + 0] = v[0]; w[4 * q + 1] = v[1]; w[4 * q + 2] = v[2]; w[4 * q + 3] = v[3];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const bool ok = rok && ks + j < g.k;
                raw[j] = ok ? (uint32_t)(uint16_t)p[ok ? ks + j : 0u] : 0u;
            }
        }
    }
    // Same tile through a buffer resource based at the block's first row (the
    // 128 rows span fewer than 2^31 bytes): an element outside the matrix gets
    // offset kOob and reads as 0, so no load needs a condition or a select.
    template <bool VEC>
    __device__ __forceinline__ void load_buf(const GemmArgs& g, __amdgpu_buffer_rsrc_t ra,
                                             uint32_t row0, uint32_t k0) {
        const uint32_t rel = a_row(threadIdx.x);
        const uint32_t ks = k0 + a_chunk(threadIdx.x) * 16;
        const bool rok = row0 + rel < g.rows;
        const uint32_t rbyte = rel * (uint32_t)g.lda * 2u;
        if constexpr (VEC) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const bool ok = rok && ks + q * 8 < g.k;
                const v4u v = __builtin_amdgcn_raw_buffer_load_b128(
                    ra, ok ? rbyte + (ks + q * 8) * 2u : kOob, 0, 0);
                w[4 * q + 0] = v[0]; w[4 * q + 1] = v[1]; w[4 * q + 2] = v[2]; w[4 * q + 3] = v[3];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const bool ok = rok && ks + j < g.k;
                raw[j] = __builtin_amdgcn_raw_buffer_load_b16(ra, ok ? rbyte + (ks + j) * 2u : kOob, 0, 0);
            }
        }
    }
    // Vector path with per-thread offsets computed once (`base`: byte offset of
    // vector q in the block's rows, kOob for rows past the end; `kc`: its k
    // within the step) and the step's k0 as the load's scalar offset: per step
    // only the k-bound test of the last, partial step costs vector work.
    __device__ __forceinline__ void load_buf_fixed(__amdgpu_buffer_rsrc_t ra, const uint32_t (&base)[2],
                                                   const uint32_t (&kc)[2], uint32_t k0, uint32_t krem) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const v4u v = __builtin_amdgcn_raw_buffer_load_b128(ra, kc[q] < krem ? base[q] : kOob,
                                                                 (int)(k0 * 2u), 0);
            w[4 * q + 0] = v[0]; w[4 * q + 1] = v[1]; w[4 * q + 2] = v[2]; w[4 * q + 3] = v[3];
        }
    }
    // Stores the limbs; hs / ls accumulate the sums of the high and low limbs
    // of this thread's values (sum a = 256*hs + ls + 128*count).
    __device__ __forceinline__ void store(bool vec, Planes& s, int32_t& hs, int32_t& ls) {
        if (!vec) {
#pragma unroll
            for (int j = 0; j < 8; ++j) w[j] = pack(raw[2 * j], raw[2 * j + 1]);
        }
        store16(s.a_hi, s.a_lo, a_off(a_row(threadIdx.x), a_chunk(threadIdx.x)), w, hs, ls);
    }
};

// ---------------------------------------------------------- dense B tile --
// Thread t owns columns [4*(t>>4), +4) and k rows [4*(t&15), +4).  Lanes of a
// wave differ mostly in k, so the transposing 4-byte LDS stores of one column
// land in 16 different banks instead of one.
struct DenseBTile {
    uint32_t w[4][2];     // [k row][word of 2 columns]
    uint32_t raw[4][4];   // element path: [k row][column], one int16 each

    __device__ __forceinline__ void load(const GemmArgs& g, const int16_t* bbase, uint32_t col0,
                                         uint32_t k0) {
        const uint32_t cb = col0 + (threadIdx.x >> 4) * 4;
        const uint32_t kb = k0 + (threadIdx.x & 15) * 4;
        if (g.b_vec) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool ok = kb + i < g.k && cb < g.cols;
                v2i v = *reinterpret_cast<const v2i*>(bbase + (ok ? (uint64_t)(kb + i) * g.ldb + cb : 0u));
                const v2i z = {0, 0};
                v = ok ? v : z;
                w[i][0] = v[0]; w[i][1] = v[1];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool kok = kb + i < g.k;
                const int16_t* p = bbase + (kok ? (uint64_t)(kb + i) * g.ldb : 0u);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const bool ok = kok && cb + q < g.cols;
                    const int16_t v = p[ok ? cb + q : 0u];
                    raw[i][q] = ok ? (uint32_t)(uint16_t)v : 0u;
                }
            }
        }
    }
    // Buffer resource based at (k0, col0) for each k step (64 rows span fewer
    // than 2^31 bytes); elements outside the matrix read as 0 through kOob.
    template <bool VEC>
    __device__ __forceinline__ void load_buf(const GemmArgs& g, __amdgpu_buffer_rsrc_t rb,
                                             uint32_t col0, uint32_t k0) {
        const uint32_t cr = (threadIdx.x >> 4) * 4;
        const uint32_t kr = (threadIdx.x & 15) * 4;
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool ok = k0 + kr + i < g.k && col0 + cr < g.cols;
                const v2u v = __builtin_amdgcn_raw_buffer_load_b64(
                    rb, ok ? ((kr + i) * (uint32_t)g.ldb + cr) * 2u : kOob, 0, 0);
                w[i][0] = v[0]; w[i][1] = v[1];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool kok = k0 + kr + i < g.k;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const bool ok = kok && col0 + cr + q < g.cols;
                    raw[i][q] = __builtin_amdgcn_raw_buffer_load_b16(
                        rb, ok ? ((kr + i) * (uint32_t)g.ldb + cr + q) * 2u : kOob, 0, 0);
                }
            }
        }
    }
    // Vector path with per-thread offsets computed once (`off`: byte offset of
    // k row i of this thread in the step's resource, kOob past the last
    // column); rows past K lie past the per-step resource and read as 0.
    __device__ __forceinline__ void load_buf_fixed(__amdgpu_buffer_rsrc_t rb, const uint32_t (&off)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const v2u v = __builtin_amdgcn_raw_buffer_load_b64(rb, off[i], 0, 0);
            w[i][0] = v[0]; w[i][1] = v[1];
        }
    }
    __device__ __forceinline__ void pack_raw() {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q) w[i][q] = pack(raw[i][2 * q], raw[i][2 * q + 1]);
    }
    // Transposes 4 k rows x 4 columns into one limb word per column: for the
    // column pair held in word q, two perms interleave rows (0,1) and (2,3),
    // two more split even / odd columns.  hs / ls accumulate per-column limb sums.
    __device__ __forceinline__ void store(Planes& s, int32_t (&hs)[4], int32_t (&ls)[4]) const {
        const uint32_t cl = (threadIdx.x >> 4) * 4;
        const uint32_t kbyte = (threadIdx.x & 15) * 4;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t t01 = __builtin_amdgcn_perm(w[1][q], w[0][q], 0x07030501u);
            const uint32_t t23 = __builtin_amdgcn_perm(w[3][q], w[2][q], 0x07030501u);
            const uint32_t u01 = __builtin_amdgcn_perm(w[1][q], w[0][q], 0x06020400u);
            const uint32_t u23 = __builtin_amdgcn_perm(w[3][q], w[2][q], 0x06020400u);
            const uint32_t hi_e = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
            const uint32_t hi_o = __builtin_amdgcn_perm(t23, t01, 0x07060302u);
            const uint32_t lo_e = __builtin_amdgcn_perm(u23, u01, 0x05040100u) ^ 0x80808080u;
            const uint32_t lo_o = __builtin_amdgcn_perm(u23, u01, 0x07060302u) ^ 0x80808080u;
            hs[2 * q] = bsum(hi_e, hs[2 * q]);
            hs[2 * q + 1] = bsum(hi_o, hs[2 * q + 1]);
            ls[2 * q] = bsum(lo_e, ls[2 * q]);
            ls[2 * q + 1] = bsum(lo_o, ls[2 * q + 1]);
            const uint32_t c = cl + 2 * q;
            *reinterpret_cast<uint32_t*>(s.b_hi + c * kStride + kbyte) = hi_e;
            *reinterpret_cast<uint32_t*>(s.b_hi + (c + 1) * kStride + kbyte) = hi_o;
            *reinterpret_cast<uint32_t*>(s.b_lo + c * kStride + kbyte) = lo_e;
            *reinterpret_cast<uint32_t*>(s.b_lo + (c + 1) * kStride + kbyte) = lo_o;
        }
    }
};

// Column sums of the dense B tile: count = k values per column this thread stored.
__device__ __forceinline__ void publish_dense(Smem& s, const int32_t (&hs)[4], const int32_t (&ls)[4],
                                              uint32_t count) {
    const uint32_t cl = (threadIdx.x >> 4) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        atomicAdd(&s.col_sum[cl + j], 256u * (uint32_t)hs[j] + (uint32_t)ls[j] + 128u * count);
}

// Eight int16 values of one output row at element offsets oc[0..7] from p:
// w-wide accesses (w = 8, 4, 2; runs of w columns are contiguous and aligned)
// when all eight columns exist, else one element per existing column (n < 8).
__device__ __forceinline__ void store8(int16_t* p, const uint64_t (&oc)[8], uint32_t n, uint32_t w,
                                       const int32_t (&y)[8]) {
    if (n == 8u && w == 8u) {
        *reinterpret_cast<v4u*>(p + oc[0]) = v4u{pack(y[0], y[1]), pack(y[2], y[3]),
                                                 pack(y[4], y[5]), pack(y[6], y[7])};
    } else if (n == 8u && w == 4u) {
        *reinterpret_cast<v2u*>(p + oc[0]) = v2u{pack(y[0], y[1]), pack(y[2], y[3])};
        *reinterpret_cast<v2u*>(p + oc[4]) = v2u{pack(y[4], y[5]), pack(y[6], y[7])};
    } else if (n == 8u && w == 2u) {
#pragma unroll
        for (int q = 0; q < 8; q += 2) *reinterpret_cast<uint32_t*>(p + oc[q]) = pack(y[q], y[q + 1]);
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q)
            if ((uint32_t)q < n) p[oc[q]] = (int16_t)y[q];
    }
}

// Adds the int16 values at the same offsets (the fused Add's tensor) to a[].
__device__ __forceinline__ void load8(const int16_t* p, const uint64_t (&oc)[8], uint32_t n, uint32_t w,
                                      int32_t (&a)[8]) {
    int32_t x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (n == 8u && w == 8u) {
        const v4u v = *reinterpret_cast<const v4u*>(p + oc[0]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            x[2 * q] = (int32_t)(int16_t)(v[q] & 0xFFFFu);
            x[2 * q + 1] = (int32_t)v[q] >> 16;
        }
    } else if (n == 8u && w == 4u) {
        const v2u v0 = *reinterpret_cast<const v2u*>(p + oc[0]);
        const v2u v1 = *reinterpret_cast<const v2u*>(p + oc[4]);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            x[2 * q] = (int32_t)(int16_t)(v0[q] & 0xFFFFu);
            x[2 * q + 1] = (int32_t)v0[q] >> 16;
            x[2 * q + 4] = (int32_t)(int16_t)(v1[q] & 0xFFFFu);
            x[2 * q + 5] = (int32_t)v1[q] >> 16;
        }
    } else if (n == 8u && w == 2u) {
#pragma unroll
        for (int q = 0; q < 8; q += 2) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(p + oc[q]);
            x[q] = (int32_t)(int16_t)(v & 0xFFFFu);
            x[q + 1] = (int32_t)v >> 16;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = p[oc[(uint32_t)q < n ? q : 0]];
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) a[q] += x[q];
}

// ------------------------------------------------------- im2col B tile --
// Thread t owns column (pixel) t&127 and k values [16*(t>>7), +16): the lanes
// of one load instruction read 64 neighbouring output pixels at the same k,
// which coalesce.  The 16 values stay raw until store().
struct ConvBTile {
    uint32_t raw[16];
    const int16_t* xb;   // image base of this thread's column
    int32_t ih0, iw0;    // window origin of this thread's output pixel
    int32_t pbase;       // ih0 * W + iw0 (may be negative; only valid taps are read)
    int32_t pbyte;       // byte offset of the window origin from the tensor start
    uint32_t holes;      // table mode: bit r set iff tap r of the window lies outside the image
    bool col_ok;

    __device__ __forceinline__ void init(const GemmArgs& g, uint32_t col0) {
        const uint32_t col = col0 + (threadIdx.x & 127);
        col_ok = col < g.cols;
        const uint32_t n = col_ok ? fdiv(col, g.div_p) : 0;
        const uint32_t p = col_ok ? col - n * g.P : 0;
        const uint32_t oh = fdiv(p, g.div_ow), ow = p - oh * g.OW;
        // a column past the end gets a window origin no tap can reach, so the
        // per-tap bounds test alone rejects it (a separate lane-varying test
        // would let the compiler branch around the gather and serialise it)
        ih0 = col_ok ? (int32_t)(oh * g.sh) - (int32_t)g.pt : 0x40000000;
        iw0 = (int32_t)(ow * g.sw) - (int32_t)g.pl;
        pbase = ih0 * (int32_t)g.W + iw0;
        pbyte = (int32_t)(2 * ((int64_t)n * (int64_t)g.x_img + pbase));
        xb = g.b + (uint64_t)n * g.x_img;
    }
    // Table mode (kh*kw <= 31): which of the window's taps r = khi*kw + kwi lie
    // outside the image (bit 31, the tap of every k >= K, is always set).
    __device__ __forceinline__ void init_taps(const GemmArgs& g) {
        uint32_t taps = 0;
        uint32_t khi = 0, kwi = 0;
        for (uint32_t r = 0; r < g.kh * g.kw; ++r) {
            const uint32_t ih = (uint32_t)(ih0 + (int32_t)(khi * g.dh));
            const uint32_t iw = (uint32_t)(iw0 + (int32_t)(kwi * g.dw));
            taps |= (ih < g.H && iw < g.W) ? 1u << r : 0u;
            if (++kwi == g.kw) { kwi = 0; ++khi; }
        }
        holes = ~taps;
    }
    // Gather through the per-block k table tab[k] = {2*(c*H*W + khi*dh*W + kwi*dw), tap r}
    // with buffer loads over the whole input tensor (fewer than 2^31 bytes):
    // the offset of a tap outside the image gets bit 31 set (its hole bit,
    // shifted), which puts it past the buffer's size, and the hardware returns
    // 0.  Three VALU operations per value, and no select the compiler could
    // turn into a branch around the table read.
    __device__ __forceinline__ void load_tab(const GemmArgs& g, uint32_t k0, const int2* tab,
                                             __amdgpu_buffer_rsrc_t rsrc) {
        // the table covers every k the loop loads, also past K (tap 31: never valid)
        const uint32_t ks = __builtin_amdgcn_readfirstlane(k0 + (threadIdx.x >> 7) * 16);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int2 t = tab[ks + j];
            const uint32_t hole = __builtin_amdgcn_ubfe(holes, (uint32_t)t.y, 1u);
            const uint32_t off = (hole << 31) | (uint32_t)(pbyte + t.x);
            raw[j] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
        }
    }
    // Gather for any size: k decomposed incrementally, global loads of a valid
    // address (element 0 of the image for invalid taps), zeroed afterwards.
    __device__ __forceinline__ void load(const GemmArgs& g, uint32_t k0) {
        const uint32_t ks = k0 + (threadIdx.x >> 7) * 16;
        const uint32_t kk = g.kh * g.kw;
        uint32_t c = fdiv(ks, g.div_kk);
        uint32_t r = ks - c * kk;
        uint32_t khi = fdiv(r, g.div_kw);
        uint32_t kwi = r - khi * g.kw;
        const uint32_t hw = g.H * g.W;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int32_t ih = ih0 + (int32_t)(khi * g.dh);
            const int32_t iw = iw0 + (int32_t)(kwi * g.dw);
            const bool ok = ks + j < g.k && (uint32_t)ih < g.H && (uint32_t)iw < g.W;
            const int16_t x = xb[ok ? (uint64_t)c * hw + (uint32_t)ih * g.W + (uint32_t)iw : 0u];
            raw[j] = ok ? (uint32_t)(uint16_t)x : 0u;
            if (++kwi == g.kw) {
                kwi = 0;
                if (++khi == g.kh) { khi = 0; ++c; }
            }
        }
    }
    __device__ __forceinline__ void store(Planes& s, int32_t& hs, int32_t& ls) const {
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = pack(raw[2 * j], raw[2 * j + 1]);
        store16(s.b_hi, s.b_lo, (threadIdx.x & 127) * kStride + (threadIdx.x >> 7) * 16, w, hs, ls);
    }
};

// B-operand modes: dense matrix, implicit-GEMM gather with an LDS k table
// (K + 2 steps <= kTabMax, at most 31 taps), implicit-GEMM gather with
// incremental k decomposition (any size).
enum { B_DENSE = 0, B_CONV_TAB = 1, B_CONV_INC = 2 };

// AV / BV: 0 = vector loads chosen at run time (g.a_vec / g.b_vec, global
// loads), 1 = vector buffer loads, 2 = element buffer loads.  Fixing the path
// at compile time keeps the staged registers identical on every path, so no
// copy (and no wait for outstanding loads) is needed where paths would merge.
template <int MODE, bool HAS_BIAS, bool FOLD, bool BUF, int AV, int BV>
__global__ __launch_bounds__(kThreads) void q88_gemm(GemmArgs g) {
    touch_lines(g);
    constexpr bool CONV = MODE != B_DENSE;
    __shared__ __align__(16) Smem s;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.y * BM;
    const uint32_t col0 = blockIdx.x * BN;
    const uint32_t wrow = (wave >> 2) * 64, wcol = (wave & 3) * 32;

    const int16_t* abase = g.a + (CONV ? 0 : (uint64_t)blockIdx.z * g.a_bs);
    const int16_t* bbase = g.b + (CONV ? 0 : (uint64_t)blockIdx.z * g.b_bs);

    if (threadIdx.x < BN) s.col_sum[threadIdx.x] = 0;   // published with atomics at the end
    if (HAS_BIAS && threadIdx.x < BM) {
        const uint32_t r = row0 + threadIdx.x;
        s.bias[threadIdx.x] = r < g.rows ? (int32_t)g.bias[r] * 256 : 0;
    }
    if (CONV && threadIdx.x >= BM && threadIdx.x < BM + BN) {
        const uint32_t col = col0 + threadIdx.x - BM;
        const uint32_t n = fdiv(col, g.div_p);
        s.coff[threadIdx.x - BM] = (uint64_t)n * g.y_img + (col - n * g.P);
    }
    const int2* tab = nullptr;
    if constexpr (MODE == B_CONV_TAB) {
        // one entry per k the main loop loads: its k steps plus the two past
        // the end (the host keeps that below kTabMax); k >= K gets tap 31
        __shared__ int2 ktab[kTabMax];
        const uint32_t kk = g.kh * g.kw, hw = g.H * g.W;
        const uint32_t kend = ((g.k + BK - 1) / BK + 2) * BK;
        for (uint32_t k = threadIdx.x; k < kend; k += kThreads) {
            const uint32_t c = fdiv(k, g.div_kk), r = k - c * kk;
            const uint32_t khi = fdiv(r, g.div_kw), kwi = r - khi * g.kw;
            const uint32_t dy = khi * g.dh, dx = kwi * g.dw;
            ktab[k] = k < g.k ? int2{(int)(2 * (c * hw + dy * g.W + dx)), (int)r} : int2{0, 31};
        }
        tab = ktab;
    }
    __syncthreads();

    // Two register stages and two LDS planes: while the MFMA phase reads the
    // planes of step k, the loads of step k+2 are in flight and step k+1 (already
    // in registers) is split into the other planes; one barrier per step.
    ATile at[2];
    using BTile = typename std::conditional<CONV, ConvBTile, DenseBTile>::type;
    BTile bt[2];
    int32_t row_hs = 0, row_ls = 0;
    int32_t dhs[4] = {0, 0, 0, 0}, dls[4] = {0, 0, 0, 0};
    int32_t chs = 0, cls = 0;
    if constexpr (CONV) {
        bt[0].init(g, col0);
        if constexpr (MODE == B_CONV_TAB) bt[0].init_taps(g);
        bt[1] = bt[0];
    }
    const __amdgpu_buffer_rsrc_t xrsrc = make_rsrc(g.b, g.x_bytes);   // table mode only
    const uint32_t arows = g.rows - row0 < (uint32_t)BM ? g.rows - row0 : (uint32_t)BM;
    const __amdgpu_buffer_rsrc_t arsrc =
        make_rsrc(abase + (uint64_t)row0 * g.lda, arows * (uint32_t)g.lda * 2u);   // BUF only

    v4i hh[TI][TJ], mid[TI][TJ], ll[TI][TJ], tot[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            hh[i][j] = v4i{0, 0, 0, 0}; mid[i][j] = v4i{0, 0, 0, 0}; ll[i][j] = v4i{0, 0, 0, 0};
            if constexpr (FOLD) tot[i][j] = v4i{0, 0, 0, 0};
        }

    // vector buffer paths: per-thread load offsets, the same for every k step
    uint32_t a_base[2], a_kc[2], b_off[4];
    {
        const uint32_t rel = a_row(threadIdx.x);
        const bool rok = row0 + rel < g.rows;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            a_kc[q] = a_chunk(threadIdx.x) * 16 + q * 8;
            a_base[q] = rok ? (rel * (uint32_t)g.lda + a_kc[q]) * 2u : kOob;
        }
        const uint32_t cr = (threadIdx.x >> 4) * 4, kr = (threadIdx.x & 15) * 4;
        const bool cok = col0 + cr < g.cols;
#pragma unroll
        for (int i = 0; i < 4; ++i) b_off[i] = cok ? ((kr + i) * (uint32_t)g.ldb + cr) * 2u : kOob;
    }
    auto load_tile = [&](ATile& a, BTile& b, uint32_t k0) {
        if constexpr (BUF && AV == 1)
            a.load_buf_fixed(arsrc, a_base, a_kc, k0, k0 < g.k ? g.k - k0 : 0u);
        else if constexpr (BUF) a.template load_buf<false>(g, arsrc, row0, k0);
        else a.load(g, abase, row0, k0);
        if constexpr (MODE == B_CONV_TAB) {
            b.load_tab(g, k0, tab, xrsrc);
        } else if constexpr (MODE == B_CONV_INC) {
            b.load(g, k0);
        } else if constexpr (BUF) {
            // k0 may lie past the last step (see the main loop): an empty resource
            const uint32_t kr = k0 >= g.k ? 0u : (g.k - k0 < (uint32_t)BK ? g.k - k0 : (uint32_t)BK);
            const uint32_t cr = g.cols - col0 < (uint32_t)BN ? g.cols - col0 : (uint32_t)BN;
            const __amdgpu_buffer_rsrc_t rb = make_rsrc(bbase + (uint64_t)(kr ? k0 : 0u) * g.ldb + col0,
                                                        kr ? ((kr - 1) * (uint32_t)g.ldb + cr) * 2u : 0u);
            if constexpr (BV == 1) b.load_buf_fixed(rb, b_off);
            else b.template load_buf<false>(g, rb, col0, k0);
        } else {
            b.load(g, bbase, col0, k0);
        }
    };
    // Splits a staged tile into planes p.  Its limb sums count only if the tile
    // is a real k step (`real`); the last step of the unrolled loop stages a
    // stale register set into planes nobody reads, without a branch, so the
    // split can interleave with the MFMA phase.
    // convolution: weight rows past the last output channel are never stored,
    // so their limbs need not be staged (uniform per wave when M % 16 == 0)
    const bool a_row_live = !CONV || row0 + a_row(threadIdx.x) < g.rows;
    auto stage_tile = [&](ATile& a, BTile& b, Planes& p, bool real) {
        int32_t h = 0, l = 0;
        if (a_row_live) a.store(AV == 0 ? g.a_vec != 0 : AV == 1, p, h, l);
        row_hs += real ? h : 0;
        row_ls += real ? l : 0;
        if constexpr (CONV) {
            int32_t ch = 0, cl = 0;
            b.store(p, ch, cl);
            chs += real ? ch : 0;
            cls += real ? cl : 0;
        } else {
            if (BUF ? BV == 2 : !g.b_vec) b.pack_raw();
            int32_t th[4] = {0, 0, 0, 0}, tl[4] = {0, 0, 0, 0};
            b.store(p, th, tl);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                dhs[j] += real ? th[j] : 0;
                dls[j] += real ? tl[j] : 0;
            }
        }
    };
    // Scheduling hint for the block of one k step: alternate each MFMA with two
    // VALU instructions of the split, so the matrix core and the vector ALU run
    // together.
    auto interleave = [&]() {
#pragma unroll
        for (int q = 0; q < TI * TJ * 4; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
        }
    };
    const bool wave_rows = row0 + wrow < g.rows;
    const bool wave_half = row0 + wrow + 32 >= g.rows;   // row tiles 2, 3 of the wave empty
    // the MFMAs of the wave's first NI row tiles (the others are left untouched)
    auto mfma_rows = [&](auto ni, const Planes& p, uint32_t it) {
        constexpr int NI = decltype(ni)::value;
        const uint32_t kq = lane >> 4;
        const uint32_t abase = a_off(wrow + (lane & 15), kq);   // wrow % 16 == 0: + i * 16 rows = + i * 256
        v4i ah[TI], al[TI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t r = abase + i * 256;
            ah[i] = *reinterpret_cast<const v4i*>(p.a_hi + r);
            al[i] = *reinterpret_cast<const v4i*>(p.a_lo + r);
        }
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const uint32_t cidx = (wcol + j * 16 + (lane & 15)) * kStride + kq * 16;
            const v4i bh = *reinterpret_cast<const v4i*>(p.b_hi + cidx);
            const v4i bl = *reinterpret_cast<const v4i*>(p.b_lo + cidx);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                hh[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bh, hh[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[i], bl, mid[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                ll[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bl, ll[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < NI; ++i)
                mid[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[i], bh, mid[i][j], 0, 0, 0);
        }

        if constexpr (FOLD) {
            if ((it + 1) % kFoldIters == 0) {
#pragma unroll
                for (int i = 0; i < TI; ++i)
#pragma unroll
                    for (int j = 0; j < TJ; ++j) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            tot[i][j][e] = (int)((uint32_t)tot[i][j][e] + ((uint32_t)hh[i][j][e] << 16) +
                                                 ((uint32_t)mid[i][j][e] << 8) + (uint32_t)ll[i][j][e]);
                        hh[i][j] = v4i{0, 0, 0, 0}; mid[i][j] = v4i{0, 0, 0, 0}; ll[i][j] = v4i{0, 0, 0, 0};
                    }
            }
        }
    };
    // convolution with few output channels: waves past the last channel skip
    // the step, waves with at most 32 live rows run half of it (uniform
    // branches; the dense GEMM keeps the single straight-line step, which
    // schedules better)
    auto mfma_step = [&](const Planes& p, uint32_t it) {
        if constexpr (CONV) {
            if (!wave_rows) return;
            if (wave_half) {
                mfma_rows(std::integral_constant<int, 2>{}, p, it);
                return;
            }
        }
        mfma_rows(std::integral_constant<int, TI>{}, p, it);
    };

    // this block's k steps: all of them, or its split's share (sums over any
    // k range obey the limb identity with that range's row / column sums and Kp)
    const uint32_t nk_all = (g.k + BK - 1) / BK;
    const uint32_t s0 = g.split_steps ? blockIdx.z * g.split_steps : 0u;
    const uint32_t nk = g.split_steps ? min(g.split_steps, nk_all - s0) : nk_all;
    const uint32_t kbase = s0 * BK;
    load_tile(at[0], bt[0], kbase);
    load_tile(at[1], bt[1], kbase + BK);
    // with K = 0 there is no step: the staged (all-zero) tile must not count,
    // its limb sums are not those of zeros (low limbs are offset by -128)
    stage_tile(at[0], bt[0], s.st[0], nk > 0);
    __syncthreads();
    // Steps go in pairs (it, it + 1).  Step it computes on planes 0 while the
    // loads of step it+2 fly into register set 0 (free: its tile was staged one
    // step earlier) and set 1 (step it+1) is split into planes 1; step it+1 is
    // the mirror image.  Loads are issued on every path, also for the (all
    // zero, out-of-range) steps past the last one, and the loop has no exit but
    // its end: a path that skips loads or leaves the loop mid-body makes the
    // compiler's wait before each split count the just-issued loads too, which
    // exposes their full latency every step.  An odd last step runs after the
    // loop from planes 0.
    uint32_t it = 0;
    for (; it + 2 <= nk; it += 2) {
        load_tile(at[0], bt[0], kbase + (it + 2) * BK);
        __builtin_amdgcn_sched_barrier(0);   // keep the loads ahead of this step's work
        mfma_step(s.st[0], it);
        stage_tile(at[1], bt[1], s.st[1], true);
        interleave();
        __syncthreads();
        load_tile(at[1], bt[1], kbase + (it + 3) * BK);
        __builtin_amdgcn_sched_barrier(0);
        mfma_step(s.st[1], it + 1);
        stage_tile(at[0], bt[0], s.st[0], it + 2 < nk);
        interleave();
        __syncthreads();
    }
    if (it < nk) mfma_step(s.st[0], it);

    // row sums (sum a = 256*hs + ls + 128*count); the four threads of a row are
    // adjacent lanes, each stored 16 k values per step
    uint32_t row_sum = 256u * (uint32_t)row_hs + (uint32_t)row_ls + 128u * 16u * nk;
    row_sum += (uint32_t)__shfl_xor((int)row_sum, 1, 64);
    row_sum += (uint32_t)__shfl_xor((int)row_sum, 2, 64);
    if (a_chunk(threadIdx.x) == 0) s.row_sum[a_row(threadIdx.x)] = row_sum;
    if constexpr (CONV)
        atomicAdd(&s.col_sum[threadIdx.x & 127], 256u * (uint32_t)chs + (uint32_t)cls + 128u * 16u * nk);
    else
        publish_dense(s, dhs, dls, 4u * nk);
    __syncthreads();   // every wave is past its last plane read: the tile may overwrite them

    // Epilogue, phase 1: each wave's MFMA sums (limb terms combined mod 2^32)
    // into the LDS tile, in the MFMA result layout (lane = column, 4 rows each).
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t v = ((uint32_t)hh[i][j][e] << 16) + ((uint32_t)mid[i][j][e] << 8) +
                             (uint32_t)ll[i][j][e];
                if constexpr (FOLD) v += (uint32_t)tot[i][j][e];
                s.tile[(wrow + i * 16 + (lane >> 4) * 4 + e) * kTilePitch + wcol + j * 16 + (lane & 15)] = v;
            }
    __syncthreads();

    // Phase 2, row-major: thread t finishes columns [c8, c8 + 8) of rows rb, rb + 32,
    // rb + 64, rb + 96 (16 threads cover a row): sum corrections, bias, saturation,
    // the fused Add and activation, then one store of the 8 values (or out_w-wide
    // pieces).  Activation and Add mode are applied without a per-value branch.
    const uint32_t c8 = (threadIdx.x & 15) * 8, rb = threadIdx.x >> 4;
    const uint32_t cbase = col0 + c8;
    if (cbase >= g.cols) return;
    const uint32_t kp_term = 16384u * (nk * (uint32_t)BK);
    uint32_t cterm[8];   // 128 * column sum - 16384 * Kp
    {
        const v4u c0 = *reinterpret_cast<const v4u*>(&s.col_sum[c8]);
        const v4u c1 = *reinterpret_cast<const v4u*>(&s.col_sum[c8 + 4]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            cterm[q] = 128u * c0[q] - kp_term;
            cterm[q + 4] = 128u * c1[q] - kp_term;
        }
    }
    auto tile_row = [&](uint32_t r, uint32_t (&v)[8]) {
        const v4u t0 = *reinterpret_cast<const v4u*>(&s.tile[r * kTilePitch + c8]);
        const v4u t1 = *reinterpret_cast<const v4u*>(&s.tile[r * kTilePitch + c8 + 4]);
        const uint32_t rs = 128u * s.row_sum[r] + (HAS_BIAS ? (uint32_t)s.bias[r] : 0u);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[q] = t0[q] + cterm[q] + rs;
            v[q + 4] = t1[q] + cterm[q + 4] + rs;
        }
    };
    if (g.ws) {   // split-K partial: raw sums; bias and epilogue in split_reduce
        uint32_t* wp = g.ws + (uint64_t)blockIdx.z * g.rows * g.ws_ld + cbase;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const uint32_t r = rb + rr * 32;
            if (row0 + r >= g.rows) break;
            uint32_t v[8];
            tile_row(r, v);
            uint32_t* p = wp + (uint64_t)(row0 + r) * g.ws_ld;   // ws_ld >= cbase + 8
            *reinterpret_cast<v4u*>(p) = v4u{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<v4u*>(p + 4) = v4u{v[4], v[5], v[6], v[7]};
        }
        return;
    }
    const uint32_t ncol = g.cols - cbase < 8u ? g.cols - cbase : 8u;
    const int32_t lo = q88::act_lo(g.epi.act), hi = q88::act_hi(g.epi.act);
    int32_t cadd[8] = {0, 0, 0, 0, 0, 0, 0, 0};   // Add of one value per column
    if (g.epi.add_mode == 2u) {
#pragma unroll
        for (int q = 0; q < 8; ++q) cadd[q] = g.epi.add[cbase + ((uint32_t)q < ncol ? q : 0)];
    }
    uint64_t ocol[8];   // output offset of each column in row 0 of the output
#pragma unroll
    for (int q = 0; q < 8; ++q) ocol[q] = CONV ? s.coff[c8 + q] : (uint64_t)(cbase + q);
    const uint64_t rstride = CONV ? (uint64_t)g.P : g.ldc;
    int16_t* cptr = g.c + (CONV ? 0 : (uint64_t)blockIdx.z * g.c_bs);
    const int16_t* rptr = g.epi.add + (CONV ? 0 : (uint64_t)blockIdx.z * g.c_bs);
    // the fused Add's values of all four rows first (rows past the end read the
    // last row), so their loads are in flight together
    int32_t add[4][8];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
#pragma unroll
        for (int q = 0; q < 8; ++q) add[rr][q] = cadd[q];
    if (g.epi.add_mode == 1u) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const uint32_t row = min(row0 + rb + rr * 32, g.rows - 1u);
            load8(rptr + (uint64_t)row * rstride, ocol, ncol, g.out_w, add[rr]);
        }
    }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const uint32_t r = rb + rr * 32;
        if (row0 + r >= g.rows) break;
        const uint64_t ro = (uint64_t)(row0 + r) * rstride;
        uint32_t v[8];
        tile_row(r, v);
        int32_t y[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) y[q] = q88::clamp(q88::add(q88::acc_to_data(v[q]), add[rr][q]), lo, hi);
        store8(cptr + ro, ocol, ncol, g.out_w, y);
    }
}

// Split-K second pass: sums the partials of four neighbouring elements of one
// output row over the splits, adds the bias, saturates, applies the epilogue
// and stores the values in the MatMul ([rows][ldc]) or convolution (NCHW)
// output layout.
constexpr int kReduceThreads = 256;
constexpr uint32_t kMaxSplits = 16;

struct ReduceArgs {
    const uint32_t* ws;      // [splits][rows][ws_ld]
    uint32_t rows, cols, ws_ld;
    FastDiv div_q;           // division by ws_ld / 4 (chunks per row)
    const int16_t* bias;
    int16_t* y;
    uint32_t conv, P;
    FastDiv div_p;
    uint64_t y_img, ldc;
    EpiArgs epi;
};

// SPLITS is a template parameter so the partial loads are unrolled and all in
// flight at once (a run-time trip count would wait for each in turn).
template <uint32_t SPLITS>
__global__ __launch_bounds__(kReduceThreads) void split_reduce(ReduceArgs a) {
    touch_lines(a);
    const uint32_t nq = a.ws_ld / 4u;
    const uint32_t total = a.rows * nq;     // < 2^20: splits need fewer than 160 output tiles
    const uint64_t zs = (uint64_t)a.rows * a.ws_ld;
    const int32_t lo = q88::act_lo(a.epi.act), hi = q88::act_hi(a.epi.act);
    for (uint32_t idx = blockIdx.x * kReduceThreads + threadIdx.x; idx < total;
         idx += gridDim.x * kReduceThreads) {
        const uint32_t row = fdiv(idx, a.div_q);
        const uint32_t c4 = (idx - row * nq) * 4u;
        if (c4 >= a.cols) continue;
        const uint32_t* src = a.ws + (uint64_t)row * a.ws_ld + c4;
        v4u part[SPLITS];
#pragma unroll
        for (uint32_t z = 0; z < SPLITS; ++z)
            part[z] = *reinterpret_cast<const v4u*>(src + z * zs);
        const uint32_t b = a.bias ? (uint32_t)(int32_t)a.bias[row] << 8 : 0u;
        v4u v = v4u{b, b, b, b};
#pragma unroll
        for (uint32_t z = 0; z < SPLITS; ++z) v += part[z];
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t col = c4 + q;
            if (col >= a.cols) break;
            uint64_t o;
            if (a.conv) {
                const uint32_t img = fdiv(col, a.div_p);
                o = (uint64_t)img * a.y_img + (uint64_t)row * a.P + (col - img * a.P);
            } else {
                o = (uint64_t)row * a.ldc + col;
            }
            int32_t yv = q88::acc_to_data(v[q]);
            if (a.epi.add_mode) yv = q88::add(yv, a.epi.add[a.epi.add_mode == 1u ? o : (uint64_t)col]);
            a.y[o] = (int16_t)q88::clamp(yv, lo, hi);
        }
    }
}

template <uint32_t S>
int launch_reduce(uint32_t splits, dim3 grid, hipStream_t s, const ReduceArgs& r) {
    if constexpr (S > kMaxSplits) {
        return cm_set_error(CM_ERR_INVALID, "split_reduce: %u splits", splits);
    } else {
        if (splits != S) return launch_reduce<S + 1>(splits, grid, s, r);
        hipLaunchKernelGGL(split_reduce<S>, grid, dim3(kReduceThreads), 0, s, r);
        return cm_check_launch("split_reduce");
    }
}

// Number of k splits for a launch of `tiles` blocks over nk_all k steps: enough
// blocks for every CU when the tile grid alone leaves most of the chip idle,
// at least two k steps per split (one when there are fewer than 64 tiles: a
// handful of blocks each walking all of K is the slowest case), at most 16.
// A split saves k steps per block but adds the reduce launch (~4-5 us); measured
// on MobileNetV2-like layers it pays from 8 k steps at 64-159 tiles, and below
// 64 tiles from 3 steps (2 when there are fewer than 20 tiles).
uint32_t choose_splits(uint32_t tiles, uint32_t nk_all) {
    if (tiles >= 160) return 1;
    if (tiles >= 64 ? nk_all < 8 : (nk_all < 2 || (nk_all == 2 && tiles >= 20))) return 1;
    const uint32_t want = (256 + tiles - 1) / tiles;
    const uint32_t cap = tiles < 64 ? nk_all : nk_all / 2;
    uint32_t sp = want < cap ? want : cap;
    if (sp > kMaxSplits) sp = kMaxSplits;
    return sp < 2 ? 1 : sp;
}

inline bool aligned(const void* p, uintptr_t n) { return ((uintptr_t)p & (n - 1)) == 0; }

template <int MODE>
int launch_gemm(GemmArgs& g0, uint32_t zdim, const LaunchCtx& lc, const char* name) {
    GemmArgs g = g0;
    const hipStream_t s = lc.s;
    dim3 grid((g.cols + BN - 1) / BN, (g.rows + BM - 1) / BM, zdim);
    if (grid.y > 65535u || grid.z > 65535u || grid.x > 0x7FFFFFFFu)
        return cm_set_error(CM_ERR_RANGE, "%s: grid too large", name);
    const bool fold = g.k > (uint32_t)(kFoldIters * BK);
    // split-K when the output tiles cannot fill the chip (single launch, no
    // fold), through the caller's workspace: the preferred split if it fits,
    // else as many splits as fit (at least two), else none
    uint32_t splits = 1;
    if (zdim == 1 && !fold) {
        const uint32_t nk_all = (g.k + BK - 1) / BK;
        splits = choose_splits(grid.x * grid.y, nk_all);
        const uint32_t ws_ld = (g.cols + 7u) & ~7u;
        const size_t per_split = (size_t)g.rows * ws_ld * 4u;
        auto even = [nk_all](uint32_t sp) {   // equal step counts: no empty split
            const uint32_t sps = (nk_all + sp - 1) / sp;
            return (nk_all + sps - 1) / sps;
        };
        if (splits > 1) splits = even(splits);
        if (lc.need) {
            const size_t want = splits > 1 ? (size_t)splits * per_split : 0u;
            if (want > *lc.need) *lc.need = want;
            return CM_OK;
        }
        // the partials are stored and summed as 16-byte vectors: a workspace that
        // is not 16-byte aligned is used from its first aligned byte on
        const uintptr_t ws_at = reinterpret_cast<uintptr_t>(lc.ws);
        const uintptr_t ws_al = (ws_at + 15u) & ~static_cast<uintptr_t>(15u);
        const size_t ws_avail = lc.ws && lc.ws_bytes > ws_al - ws_at ? lc.ws_bytes - (ws_al - ws_at) : 0u;
        if (splits > 1) {
            const size_t fit = ws_avail / per_split;
            if (fit < splits) splits = fit >= 2 ? even((uint32_t)fit) : 1u;
        }
        if (splits > 1) {
            g.split_steps = (nk_all + splits - 1) / splits;
            g.ws_ld = ws_ld;
            g.ws = reinterpret_cast<uint32_t*>(ws_al);
            g.a_bs = g.b_bs = g.c_bs = 0;
            grid.z = splits;
        }
    } else if (lc.need) {
        return CM_OK;
    }
    const bool bias = g.bias != nullptr && splits == 1;
    // widest output / Add access that keeps alignment and stays in one image row run
    g.out_w = 8;
    const bool add_same = g.epi.add_mode == 1u;
    while (g.out_w > 1u) {
        const uint32_t w = g.out_w;
        const bool ok = (MODE == B_DENSE ? g.ldc % w == 0 && (grid.z == 1 || g.c_bs % w == 0)
                                         : g.P % w == 0) &&
                        aligned(g.c, 2u * w) && (!add_same || aligned(g.epi.add, 2u * w));
        if (ok) break;
        g.out_w = w / 2u;
    }
    // Buffer loads need each per-block resource below 2^31 bytes: 128 rows of A
    // and 64 k rows of dense B.  The table-gather conv always satisfies it.
    const bool buf = MODE == B_CONV_TAB ||
                     (MODE == B_DENSE && !fold && g.lda < (1ull << 23) && g.ldb < (1ull << 24) - 128);
#define CM_GEMM_LAUNCH(B, F, U, AV, BV) \
    hipLaunchKernelGGL((q88_gemm<MODE, B, F, U, AV, BV>), grid, dim3(kThreads), 0, s, g)
#define CM_GEMM_BIAS(F, U, AV, BV) \
    do { if (bias) CM_GEMM_LAUNCH(true, F, U, AV, BV); else CM_GEMM_LAUNCH(false, F, U, AV, BV); } while (0)
    if constexpr (MODE == B_CONV_TAB) {
        if (g.a_vec) CM_GEMM_BIAS(false, true, 1, 0); else CM_GEMM_BIAS(false, true, 2, 0);
    } else if constexpr (MODE == B_DENSE) {
        if (buf) {
            if (g.a_vec) {
                if (g.b_vec) CM_GEMM_BIAS(false, true, 1, 1); else CM_GEMM_BIAS(false, true, 1, 2);
            } else {
                if (g.b_vec) CM_GEMM_BIAS(false, true, 2, 1); else CM_GEMM_BIAS(false, true, 2, 2);
            }
        } else if (fold) {
            CM_GEMM_BIAS(true, false, 0, 0);
        } else {
            CM_GEMM_BIAS(false, false, 0, 0);
        }
    } else {
        if (fold) CM_GEMM_BIAS(true, false, 0, 0); else CM_GEMM_BIAS(false, false, 0, 0);
    }
#undef CM_GEMM_BIAS
#undef CM_GEMM_LAUNCH
    if (splits == 1) return cm_check_launch(name);
    const int rc = cm_check_launch(name);
    if (rc) return rc;
    ReduceArgs r{};
    r.ws = g.ws; r.rows = g.rows; r.cols = g.cols; r.ws_ld = g.ws_ld;
    r.div_q = make_fastdiv(g.ws_ld / 4u);
    r.bias = g.bias; r.y = g.c;
    r.conv = MODE != B_DENSE; r.P = g.P; r.div_p = g.div_p;
    r.y_img = g.y_img; r.ldc = g.ldc; r.epi = g.epi;
    const uint64_t chunks = (uint64_t)g.rows * (g.ws_ld / 4u);
    const dim3 rgrid((uint32_t)cm_grid_blocks(chunks, kReduceThreads, 4096));
    return launch_reduce<2>(splits, rgrid, s, r);
}

}  // namespace

int cm_matmul_rk_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k, uint32_t m,
                        uint32_t lda, uint32_t ldc, const cm_epilogue_t* epi, const LaunchCtx& lc);
int cm_gemm_dma_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                       uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs,
                       const cm_epilogue_t* epi, const LaunchCtx& lc);

int cm_matmul_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                     uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs,
                     const cm_epilogue_t* epi, const LaunchCtx& lc) {
    if (batch == 0 || n == 0 || m == 0) return CM_OK;
    GemmArgs g{};
    g.a = a; g.b = b; g.c = c; g.bias = nullptr;
    g.epi = cm_epi_args(epi);
    g.rows = n; g.cols = m; g.k = k;
    g.lda = k; g.ldb = m; g.ldc = m;
    g.a_bs = a_bs; g.b_bs = b_bs; g.c_bs = c_bs;
    g.a_vec = aligned(a, 16) && k % 8 == 0 && a_bs % 8 == 0;
    g.b_vec = aligned(b, 8) && m % 4 == 0 && b_bs % 4 == 0;
    if (c_bs == 0 && batch > 1) {
        // every batch step overwrites the same C; the sequential reference leaves the last one
        g.a = a + (uint64_t)(batch - 1) * a_bs;
        g.b = b + (uint64_t)(batch - 1) * b_bs;
        g.a_vec = aligned(g.a, 16) && k % 8 == 0;
        g.b_vec = aligned(g.b, 8) && m % 4 == 0;
        batch = 1;
    }
    // one small product: the register-only kernel, the reduction split over a
    // block's waves (matmul_rk.hip)
    if (batch == 1) {
        const int rc = cm_matmul_rk_launch(g.a, g.b, g.c, n, k, m, k, m, epi, lc);
        if (rc != 1) return rc;
    }
    // a batch of single-row products sharing one B (the scheduler's row-strided
    // form of a product whose output rows are padded, nodes.py:785-801) is one
    // product of `batch` rows, A rows a_bs apart and C rows c_bs apart, when no
    // two batches' outputs overlap
    if (batch > 1 && n == 1 && b_bs == 0 && a_bs >= k && c_bs >= m) {
        const int rc = cm_matmul_rk_launch(a, b, c, batch, k, m, a_bs, c_bs, epi, lc);
        if (rc != 1) return rc;
    }
    // large products with a workspace for the packed B: operands streamed into
    // LDS by direct-to-LDS loads (gemm_dma.hip)
    {
        const int rc = cm_gemm_dma_launch(g.a, g.b, g.c, n, k, m, batch, a_bs, b_bs, c_bs, epi, lc);
        if (rc != 1) return rc;
    }
    // Batches whose outputs overlap (0 < c_stride < n*m) run one launch each, in
    // batch order: the reference's sequential batch loop (MatmulKernel.cpp:108-111)
    // leaves each shared element with the last batch's value.
    const bool overlap = c_bs != 0 && (uint64_t)c_bs < (uint64_t)n * m;
    const uint32_t zmax = overlap ? 1u : 65535u;   // grid.z holds at most 65535 batches
    uint32_t done = 0;
    while (done < batch) {
        const uint32_t z = (batch - done) > zmax ? zmax : (batch - done);
        GemmArgs gz = g;
        gz.a = g.a + (uint64_t)done * a_bs;
        gz.b = g.b + (uint64_t)done * b_bs;
        gz.c = g.c + (uint64_t)done * c_bs;
        if (g.epi.add_mode == 1u) gz.epi.add = g.epi.add + (uint64_t)done * c_bs;
        const int rc = launch_gemm<B_DENSE>(gz, z, lc, "matmul");
        if (rc) return rc;
        done += z;
    }
    return CM_OK;
}

int cm_conv_gemm_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                        uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                        uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                        uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                        uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc) {
    const uint64_t P = (uint64_t)out_h * out_w;
    const uint64_t K = (uint64_t)in_ch * kh * kw;
    const uint64_t cols = P * batch;
    const uint64_t x_img = (uint64_t)in_ch * in_h * in_w;
    if (cols == 0 || out_ch == 0) return CM_OK;
    if (cols > 0x7FFFFFFFull || K > 0x7FFFFFFFull || x_img > 0x7FFFFFFFull || P > 0x7FFFFFFFull)
        return cm_set_error(CM_ERR_RANGE, "conv: shape exceeds 32-bit indexing");
    GemmArgs g{};
    g.a = w; g.b = x; g.c = y; g.bias = bias;
    g.epi = cm_epi_args(epi);
    g.rows = out_ch; g.cols = (uint32_t)cols; g.k = (uint32_t)K;
    g.lda = K;
    g.a_vec = aligned(w, 16) && K % 8 == 0;
    g.b_vec = 0;
    g.C = in_ch; g.H = in_h; g.W = in_w; g.OW = out_w; g.P = (uint32_t)P;
    g.kh = kh; g.kw = kw; g.sh = sh; g.sw = sw; g.dh = dh; g.dw = dw; g.pt = pad_top; g.pl = pad_left;
    g.x_img = x_img;
    g.y_img = (uint64_t)out_ch * P;
    g.div_p = make_fastdiv((uint32_t)P);
    g.div_ow = make_fastdiv(out_w);
    g.div_kk = make_fastdiv(kh * kw);
    g.div_kw = make_fastdiv(kw);
    const uint64_t x_bytes = 2 * x_img * batch;
    g.x_bytes = (uint32_t)(x_bytes < 0x80000000ull ? x_bytes : 0);
    // table mode: at most 31 taps (one bit each), byte offsets of the window
    // below 2^31
    const bool table = ((K + BK - 1) / BK + 2) * BK <= kTabMax && (uint64_t)kh * kw <= 31u &&
                       x_bytes < 0x80000000ull &&
                       ((uint64_t)(kh - 1) * dh * in_w + (uint64_t)(kw - 1) * dw) < (1ull << 29);
    if (table) return launch_gemm<B_CONV_TAB>(g, 1, lc, "conv_gemm");
    return launch_gemm<B_CONV_INC>(g, 1, lc, "conv_gemm");
}

int cm_conv_pointwise_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                             uint32_t batch, uint32_t in_ch, uint32_t out_ch, uint32_t hw,
                             const cm_epilogue_t* epi, const LaunchCtx& lc) {
    // 1x1, stride 1, no padding: y[n] = W[out_ch][in_ch] x X[n][in_ch][hw] (+ bias)
    if (batch == 0 || out_ch == 0 || hw == 0) return CM_OK;
    GemmArgs g{};
    g.a = w; g.b = x; g.c = y; g.bias = bias;
    g.epi = cm_epi_args(epi);
    g.rows = out_ch; g.cols = hw; g.k = in_ch;
    g.lda = in_ch; g.ldb = hw; g.ldc = hw;
    g.a_bs = 0; g.b_bs = (uint64_t)in_ch * hw; g.c_bs = (uint64_t)out_ch * hw;
    g.a_vec = aligned(w, 16) && in_ch % 8 == 0;
    g.b_vec = aligned(x, 8) && hw % 4 == 0 && g.b_bs % 4 == 0;
    uint32_t done = 0;
    while (done < batch) {
        const uint32_t z = (batch - done) > 65535u ? 65535u : (batch - done);
        GemmArgs gz = g;
        gz.b = x + (uint64_t)done * g.b_bs;
        gz.c = y + (uint64_t)done * g.c_bs;
        if (g.epi.add_mode == 1u) gz.epi.add = g.epi.add + (uint64_t)done * g.c_bs;
        const int rc = launch_gemm<B_DENSE>(gz, z, lc, "conv_pointwise");
        if (rc) return rc;
        done += z;
    }
    return CM_OK;
}
