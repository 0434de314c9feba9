// pool.hip -- PoolingKernel for gfx950 (kernels/pool/kernel/PoolingKernel.cpp:37-275).
//
// MAX / AVG / LP(p=1,2) over NCHW planes with stride, dilation, top/left
// padding (bottom/right implicit through the bounds check) and
// count_include_pad.  Arithmetic per output (PoolingKernel.cpp:120-265):
//   MAX  max over the window, padded positions count as -32768 (kDataMin);
//   AVG  S = sum(x << 8) mod 2^32, out = AccData_t((float)S * fl32(1/d));
//   LP1  sum(|x| << 8) mod 2^32, saturate_cast;
//   LP2  A = sum(x^2) mod 2^32, out = AccData_t(sqrtf((float)A)).
//
// Three launch shapes, all HBM streaming (each input byte read once):
//   * global: window == whole plane (Global*Pool): one wavefront per plane,
//     8 independent 16-byte loads in flight per lane, cross-lane reduction;
//   * band:   a block stages the input rows that a band of output rows needs
//     in LDS (16-byte loads, all issued before any is consumed), then
//     computes the band from LDS;
//   * direct: rows too wide for LDS -- each thread reads its window from HBM.
// The reduction kind is a template parameter, so the inner loops carry no
// per-element type dispatch.
#include "cm_internal.h"
#include "q88.h"

#include <algorithm>

namespace {

typedef short v8s __attribute__((ext_vector_type(8)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kNonTemporal = 2;   // buffer access cache policy: nt
constexpr uint64_t kPoolBlocks = 2048;   // fallback: 256 CUs x 8 resident blocks of 256 threads

struct PoolGeom {
    uint32_t in_h, in_w, out_h, out_w, ph, pw, sh, sw, pt, pl, dh, dw;
    uint32_t pool_type, lp_order, cip;
};

// Reduction kinds: pool_type MAX, AVG, or Lp with p = 1 / 2.
enum Kind { K_MAX = 0, K_AVG = 1, K_LP1 = 2, K_LP2 = 3 };

// Accumulator for one output: uint32 wrapping sum (AVG, LP) or int32 max,
// initialised like PoolingKernel.cpp:185-190 (kAccMin = raw -2^31 for MAX).
template <int KIND>
struct Acc {
    // A padded tap: kDataMin for MAX (PoolingKernel pads with it; the result
    // equals skipping the tap, since the initial accumulator is lower), 0 for sums.
    static constexpr int32_t kPad = KIND == K_MAX ? -32768 : 0;
    uint32_t v;
    __device__ __forceinline__ Acc() : v(KIND == K_MAX ? 0x80000000u : 0u) {}
    __device__ __forceinline__ void add(int32_t x) {
        if constexpr (KIND == K_MAX) v = (uint32_t)__builtin_elementwise_max((int32_t)v, x << 8);
        else if constexpr (KIND == K_AVG) v += (uint32_t)x << 8;
        else if constexpr (KIND == K_LP1) v += (uint32_t)__builtin_abs(x) << 8;
        else v += (uint32_t)(x * x);
    }
    __device__ __forceinline__ void merge(uint32_t o) {
        if constexpr (KIND == K_MAX) v = (uint32_t)__builtin_elementwise_max((int32_t)v, (int32_t)o);
        else v += o;
    }
    // PoolingKernel.cpp:253-266
    __device__ __forceinline__ int16_t finish(float inv) const {
        if constexpr (KIND == K_AVG) return q88::avg_finalize(v, inv);
        else if constexpr (KIND == K_LP2) return q88::lp2_finalize(v);
        else return q88::acc_to_data(v);
    }
};

// Number of taps t < k with 0 <= base + t*d < lim.
__device__ __forceinline__ int32_t valid_taps(int32_t base, int32_t k, int32_t d, int32_t lim) {
    int32_t n = 0;
    for (int32_t t = 0; t < k; ++t) n += ((uint32_t)(base + t * d) < (uint32_t)lim) ? 1 : 0;
    return n;
}

// The wave's index in the block as a value the compiler knows is uniform: a
// buffer descriptor built from threadIdx.x >> 6 otherwise sits in vector
// registers, and every buffer load through it becomes a read-first-lane loop.
__device__ __forceinline__ uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Merges of Acc values across lanes by DPP: row16_reduce leaves each 16-lane
// row's merge in the row's last lane (row shifts by 1, 2, 4 and 8, the row's
// first lanes taking the merge's identity); wave_reduce merges the four row
// results read out with readlane (scalar, no LDS round trips).
template <int KIND>
__device__ __forceinline__ uint32_t acc_merge(uint32_t a, uint32_t b) {
    Acc<KIND> t;
    t.v = a;
    t.merge(b);
    return t.v;
}
template <int KIND>
__device__ __forceinline__ uint32_t row16_reduce(uint32_t v) {
    constexpr int kId = KIND == K_MAX ? (int)0x80000000u : 0;
    v = acc_merge<KIND>(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x111, 0xF, 0xF, false));
    v = acc_merge<KIND>(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x112, 0xF, 0xF, false));
    v = acc_merge<KIND>(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x114, 0xF, 0xF, false));
    v = acc_merge<KIND>(v, (uint32_t)__builtin_amdgcn_update_dpp(kId, (int)v, 0x118, 0xF, 0xF, false));
    return v;
}
template <int KIND>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v) {
    v = row16_reduce<KIND>(v);
    uint32_t t = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
    t = acc_merge<KIND>(t, (uint32_t)__builtin_amdgcn_readlane((int)v, 31));
    t = acc_merge<KIND>(t, (uint32_t)__builtin_amdgcn_readlane((int)v, 47));
    return acc_merge<KIND>(t, (uint32_t)__builtin_amdgcn_readlane((int)v, 63));
}

// ---------------------------------------------------------------- global --
// One wavefront per plane, NB 16-byte loads per lane in flight (NB fitted to the
// plane on the host: 1, 2, 4, or 8 repeated).  Each 16-byte vector (8 values, 4
// packed pairs) is reduced on the raw values: sums of x (AVG) and x^2 (LP p=2)
// by v_dot2 on the pairs, maxima by the packed 16-bit max, |x| (LP p=1) value by
// value; the int32 sums wrap, and (sum of x) << 8 equals the sum of x << 8
// modulo 2^32, so shifting once at the end gives the reference accumulator.
template <int KIND>
struct RawAcc {
    typedef short v2s __attribute__((ext_vector_type(2)));
    uint32_t s = KIND == K_MAX ? 0x80008000u : 0u;   // MAX: two packed int16 maxima
    __device__ __forceinline__ void add_pair(uint32_t w) {
        if constexpr (KIND == K_MAX) {
            s = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(v2s, s),
                                                                       __builtin_bit_cast(v2s, w)));
        } else if constexpr (KIND == K_AVG) {
            s = (uint32_t)__builtin_amdgcn_sdot2(__builtin_bit_cast(v2s, w), v2s{1, 1}, (int32_t)s, false);
        } else if constexpr (KIND == K_LP1) {
            s += (uint32_t)__builtin_abs((int32_t)(int16_t)(w & 0xFFFFu)) + (uint32_t)__builtin_abs((int32_t)w >> 16);
        } else {
            const v2s p = __builtin_bit_cast(v2s, w);
            s = (uint32_t)__builtin_amdgcn_sdot2(p, p, (int32_t)s, false);
        }
    }
    __device__ __forceinline__ void add_one(int32_t x) { add_pair(KIND == K_MAX ? ((uint32_t)x & 0xFFFFu) | 0x80000000u
                                                                                 : (uint32_t)x & 0xFFFFu); }
    // the reference accumulator (Acc<KIND>::v) of this lane's values
    __device__ __forceinline__ uint32_t acc() const {
        if constexpr (KIND == K_MAX) {
            const int32_t lo = (int32_t)(int16_t)(s & 0xFFFFu), hi = (int32_t)s >> 16;
            return (uint32_t)__builtin_elementwise_max(lo, hi) << 8;
        } else if constexpr (KIND == K_LP2) {
            return s;
        } else {
            return s << 8;
        }
    }
};

template <int KIND, int NB>
__global__ __launch_bounds__(kThreads) void pool_global(const int16_t* __restrict__ x,
                                                        int16_t* __restrict__ y, uint64_t planes,
                                                        uint32_t hw, float inv, uint32_t vec_ok) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t plane = (uint64_t)blockIdx.x * (kThreads / 64) + wave_id();
    if (plane >= planes) return;
    const int16_t* xp = x + plane * hw;
    RawAcc<KIND> r;
    uint32_t done = 0;
    if (vec_ok) {
        // range-checked buffer loads: past the plane they read 0 and touch no
        // memory, so none needs a branch and all NB are in flight together
        // (a guarded load became a branch with a wait for every earlier load);
        // 0 adds nothing to a sum, and MAX replaces those vectors by -32768
        const uint32_t nv = hw / 8;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(xp, nv * 16u);
        for (uint32_t base = 0; base < nv; base += 64 * NB) {
            v4u t[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u)
                t[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, (base + u * 64 + lane) * 16u, 0, kNonTemporal);
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const bool in = base + u * 64 + lane < nv;
#pragma unroll
                for (int j = 0; j < 4; ++j) r.add_pair(KIND == K_MAX && !in ? 0x80008000u : t[u][j]);
            }
        }
        done = nv * 8;
    }
    for (uint32_t i = done + lane; i < hw; i += 64) r.add_one(xp[i]);
    Acc<KIND> a;
    a.v = wave_reduce<KIND>(r.acc());
    if (lane == 0) y[plane] = a.finish(inv);
}

// Small planes (at most 16 * NL elements, e.g. a 7x7 GlobalAveragePool): sixteen
// lanes per plane, four planes per wave, NL two-byte loads per lane (all issued
// before any is used; positions past the plane take the pad value), the sixteen
// lanes' accumulators merged by DPP row shifts, and the group's last lane
// finishes its plane.
template <int KIND, int NL>
__global__ __launch_bounds__(kThreads) void pool_gsmall(const int16_t* __restrict__ x,
                                                        int16_t* __restrict__ y, uint64_t planes,
                                                        uint32_t hw, float inv) {
    const uint32_t lane = threadIdx.x & 63, grp = lane >> 4, j = lane & 15;
    const uint64_t plane0 = ((uint64_t)blockIdx.x * (kThreads / 64) + wave_id()) * 4;
    if (plane0 >= planes) return;
    const uint32_t np = (uint32_t)(planes - plane0 < 4 ? planes - plane0 : 4);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + plane0 * hw, np * hw * 2u);
    uint32_t v[NL];
#pragma unroll
    for (int u = 0; u < NL; ++u) {
        const uint32_t e = j + 16u * u;
        v[u] = __builtin_amdgcn_raw_buffer_load_b16(rx, e < hw ? (grp * hw + e) * 2u : kOob, 0, kNonTemporal);
    }
    Acc<KIND> a;
#pragma unroll
    for (int u = 0; u < NL; ++u) {
        const uint32_t e = j + 16u * u;
        a.add(e < hw ? (int32_t)(int16_t)v[u] : Acc<KIND>::kPad);
    }
    a.v = row16_reduce<KIND>(a.v);
    if (j == 15u && grp < np) y[plane0 + grp] = a.finish(inv);
}

// ------------------------------------------------------------------ band --
// Work item = (plane, band of `band_h` output rows).  The block stages the
// band's whole window footprint in LDS *including the padding*: rows
// [ih_lo, ih_hi] and columns [-pl, in_w + pr), padded positions holding the
// pad value (kDataMin for MAX, 0 for sums; PoolingKernel.cpp:168-172), so
// every window reads LDS without a bounds check.  LDS element (r, c) holds
// input (ih_lo + r, c - cofs); cofs >= pl is a multiple of 8 so that the
// 16-byte body of each staged input row is aligned, and the row pitch is a
// multiple of 8 elements.
//
// Blocks are persistent and software-pipelined: the 16-byte loads of the
// next item are issued into registers before the current item is reduced,
// so HBM traffic continues while windows are computed.  Each thread owns a
// fixed (row, column) of a pass of `rows_pp` output rows, computed once.
//
// `vec` (in_w % 8 == 0, 16-byte aligned planes) selects 16-byte row copies;
// otherwise rows are copied element by element.  KH/KW > 0 fix the window at
// compile time (dilation 1) so the taps unroll with immediate LDS offsets.
constexpr uint32_t kBandBytes = 8192;   // input bytes one item fetches at most (16 B per load)
#ifndef CM_POOL_BAND_TARGET
#define CM_POOL_BAND_TARGET (16u << 10)
#endif
// LDS bytes of input a band aims for: smaller bands give each persistent block
// more items to pipeline and a shorter last item
constexpr uint32_t kBandTarget = CM_POOL_BAND_TARGET < kBandBytes ? CM_POOL_BAND_TARGET : kBandBytes;
// Persistent band / strip blocks per CU, at most.  The occupancy query allows
// 8 blocks of these kernels per CU; 6 measured ~12 % faster on 32 MB tensors
// (5 and 8 slower): blocks then hold more items, so more of each item's load
// latency hides behind the previous item's reduction.
#ifndef CM_POOL_PERSIST_PER_CU
#define CM_POOL_PERSIST_PER_CU 6
#endif
constexpr int kPersistPerCu = CM_POOL_PERSIST_PER_CU;
constexpr uint32_t kInvTab = 64;   // AVG: 1/d for every denominator d <= 63, per block

struct BandGeom {
    uint32_t band_h, n_bands, n_items;
    uint32_t pitch, cofs, lds_rows;    // LDS tile: lds_rows x pitch elements (+ slack rows)
    uint32_t alloc_rows;               // rows allocated (slack for the last strip's reads)
    uint32_t vec;                      // 16-byte row copies
    uint32_t span;                     // rows not 16-byte aligned: 16-byte loads of the
                                       // aligned span around an item's rows, scattered
    uint32_t x_bytes;                  // span loads: bytes of x rounded up to 16 (the buffer range)
    uint32_t n_strips;                 // pool_strip: strips of kStrip output rows per band
    FastDiv div_w;                     // division by in_w (element copies)
};

struct BandItem {
    uint64_t plane;
    uint32_t oh0, oh1;
    int32_t ih_lo;        // input row of LDS row 0 (may be negative: top padding)
    uint32_t r0, r1;      // LDS rows [r0, r1) hold real input rows
};

__device__ __forceinline__ BandItem band_item(const PoolGeom& g, const BandGeom& b, uint32_t item) {
    BandItem it;
    it.plane = b.n_bands == 1 ? item : item / b.n_bands;
    const uint32_t band = item - (uint32_t)(it.plane * b.n_bands);
    it.oh0 = band * b.band_h;
    it.oh1 = min(it.oh0 + b.band_h, g.out_h);
    it.ih_lo = (int32_t)(it.oh0 * g.sh) - (int32_t)g.pt;
    const int32_t last = (int32_t)((it.oh1 - 1) * g.sh) - (int32_t)g.pt + (int32_t)((g.ph - 1) * g.dh);
    const int32_t lo = it.ih_lo < 0 ? 0 : it.ih_lo;
    const int32_t hi = last + 1 > (int32_t)g.in_h ? (int32_t)g.in_h : last + 1;
    it.r0 = (uint32_t)(lo - it.ih_lo);
    it.r1 = hi > lo ? (uint32_t)(hi - it.ih_lo) : it.r0;
    return it;
}

// Output rows per thread on the strip path (fixed window, row stride SH).
constexpr int kStrip = 4;

// Row partial of a KW-wide window (KW = 2 or 3) starting at LDS element p, in
// the accumulator form of Acc<KIND> (MAX: max << 8; sums wrap mod 2^32).  The
// taps are read as one aligned 4-byte pair plus at most one single value:
// `odd` says p itself is not 4-byte aligned.  Sums go through v_dot2 on the
// packed pair (x0*1 + x1*1, or x0*x0 + x1*x1 for p = 2), wrapping like the
// reference's accumulator; shifting a sum by 8 afterwards equals summing the
// shifted taps modulo 2^32.
template <int KIND, int KW>
__device__ __forceinline__ uint32_t row_window(const int16_t* p, bool odd) {
    typedef short v2s __attribute__((ext_vector_type(2)));
    uint32_t pair, single = 0;
    bool has_single = KW == 3;
    if (odd) {
        pair = *reinterpret_cast<const uint32_t*>(p + 1);
        single = (uint32_t)(int32_t)p[0];
        if (KW == 2) { pair = (pair << 16) | (single & 0xFFFFu); has_single = false; }
    } else {
        pair = *reinterpret_cast<const uint32_t*>(p);
        if (KW == 3) single = (uint32_t)(int32_t)p[2];
    }
    const int32_t s1 = has_single ? (int32_t)single : 0;
    const v2s pv = __builtin_bit_cast(v2s, pair);
    if constexpr (KIND == K_MAX) {
        const int32_t lo = (int32_t)(int16_t)(pair & 0xFFFFu), hi = (int32_t)pair >> 16;
        const int32_t m = has_single ? __builtin_elementwise_max(__builtin_elementwise_max(lo, hi), s1)
                                     : __builtin_elementwise_max(lo, hi);
        return (uint32_t)m << 8;
    } else if constexpr (KIND == K_AVG) {
        return (uint32_t)__builtin_amdgcn_sdot2(pv, __builtin_bit_cast(v2s, 0x00010001u), s1, false) << 8;
    } else if constexpr (KIND == K_LP1) {
        const int32_t lo = (int32_t)(int16_t)(pair & 0xFFFFu), hi = (int32_t)pair >> 16;
        return ((uint32_t)__builtin_abs(lo) + (uint32_t)__builtin_abs(hi) + (uint32_t)__builtin_abs(s1)) << 8;
    } else {
        return (uint32_t)__builtin_amdgcn_sdot2(pv, pv, s1 * s1, false);
    }
}

// KH/KW > 0: window fixed at compile time (dilation 1).  SH > 0 (with KH > 0):
// row stride fixed too, and each thread reduces a vertical strip of kStrip
// outputs of one column: every input row of the strip is reduced across the
// window's columns once, and each output merges KH of those row partials
// (max and the wrapping sums are associative, so the result is the same as
// tap-by-tap accumulation).  Otherwise one output per thread and pass.
template <int KIND, int KH, int KW, int SH, int PAIR>
__global__ __launch_bounds__(kThreads) void pool_band(const int16_t* __restrict__ x,
                                                      int16_t* __restrict__ y, PoolGeom g,
                                                      BandGeom b, float inv_full) {
    touch_lines(g, b);
    extern __shared__ __align__(16) int16_t lds[];
    __shared__ float inv_tab[kInvTab];
    constexpr int16_t kPadV = KIND == K_MAX ? (int16_t)-32768 : (int16_t)0;
    constexpr bool STRIP = KH > 0 && SH > 0;
    constexpr int PRE = kBandBytes / (kThreads * 16);   // 16-byte loads per thread and item
    const int32_t ph = KH > 0 ? KH : (int32_t)g.ph, pw = KW > 0 ? KW : (int32_t)g.pw;
    const int32_t dh = KH > 0 ? 1 : (int32_t)g.dh, dw = KW > 0 ? 1 : (int32_t)g.dw;
    const bool avg_tab = KIND == K_AVG && !g.cip && (uint32_t)(ph * pw) < kInvTab;
    if (KIND == K_AVG && threadIdx.x < kInvTab) inv_tab[threadIdx.x] = q88::inv_denom(threadIdx.x);

    // left [0, cofs) and right [cofs + in_w, pitch) columns are padding in every
    // row of every item (data rows only write [cofs, cofs + in_w)): filled once
    {
        const uint32_t rcols = b.pitch - b.cofs - g.in_w;
        const uint32_t strip = b.cofs + rcols;
        if (strip) {
            const uint32_t n = b.alloc_rows * strip;
            for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
                const uint32_t r = i / strip, c = i - r * strip;
                lds[r * b.pitch + (c < b.cofs ? c : c + g.in_w)] = kPadV;
            }
        }
    }

    // this thread's 16-byte vectors u: row (relative to the item's first real
    // row) and vector column, the same for every item
    const uint32_t vpr = g.in_w / 8;                 // 16-byte vectors per input row (vec path)
    uint32_t vslot[PRE];   // LDS element offset of vector u, relative to the item's row r0
#pragma unroll
    for (int u = 0; u < PRE; ++u) {
        const uint32_t v = u * kThreads + threadIdx.x;
        const uint32_t r = b.vec ? v / vpr : 0u;
        vslot[u] = r * b.pitch + b.cofs + (v - r * vpr) * 8;
    }
    const uint32_t my_r = threadIdx.x / g.out_w;          // this thread's row (strip) within a pass ...
    const uint32_t my_c = threadIdx.x - my_r * g.out_w;   // ... and column (when out_w <= 256)
    const uint32_t rows_pp = g.out_w >= (uint32_t)kThreads ? 1u : (uint32_t)kThreads / g.out_w;
    const uint32_t cstep = g.out_w > kThreads ? kThreads : g.out_w;

    // fetch: the real input rows of an item into registers (span: the 16-byte
    // vectors that cover them, one more than a row-aligned copy at most)
    v8s pre[PRE + 1];
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(x, b.span ? b.x_bytes : 0u);
    auto span_first = [&](const BandItem& it) {   // element index of the item's first real input
        return it.plane * (uint64_t)g.in_h * g.in_w + (uint64_t)(it.ih_lo + (int32_t)it.r0) * g.in_w;
    };
    auto fetch = [&](const BandItem& it) {
        if (b.span) {
            const uint64_t f0 = span_first(it), f1 = f0 + (uint64_t)(it.r1 - it.r0) * g.in_w;
            const uint64_t v0 = f0 >> 3;
            const uint32_t nv = (uint32_t)(((f1 + 7) >> 3) - v0);
#pragma unroll
            for (int u = 0; u < PRE + 1; ++u) {
                const uint32_t v = u * kThreads + threadIdx.x;
                if (v < nv)
                    pre[u] = __builtin_bit_cast(v8s, __builtin_amdgcn_raw_buffer_load_b128(
                                                         xrs, (uint32_t)((v0 + v) * 16u), 0, kNonTemporal));
            }
            return;
        }
        if (!b.vec) return;
        const int16_t* xp = x + it.plane * (uint64_t)g.in_h * g.in_w;
        const uint32_t nv = (it.r1 - it.r0) * vpr;
        const v8s* sv = reinterpret_cast<const v8s*>(xp + (int64_t)(it.ih_lo + (int32_t)it.r0) * g.in_w);
#pragma unroll
        for (int u = 0; u < PRE; ++u) {
            const uint32_t v = u * kThreads + threadIdx.x;
            if (v < nv) pre[u] = __builtin_nontemporal_load(sv + v);
        }
    };

    uint32_t item = blockIdx.x;
    if (item >= b.n_items) return;
    BandItem cur = band_item(g, b, item);
    fetch(cur);
    for (;;) {
        const uint32_t next = item + gridDim.x;
        __syncthreads();                       // the previous item's LDS reads are done
        {
            // whole padding rows outside [r0, r1) (full pitch), then the data
            const uint32_t top = cur.r0 * b.pitch;
            const uint32_t bottom = (b.lds_rows - cur.r1) * b.pitch;
            for (uint32_t i = threadIdx.x; i < top; i += kThreads) lds[i] = kPadV;
            for (uint32_t i = threadIdx.x; i < bottom; i += kThreads) lds[cur.r1 * b.pitch + i] = kPadV;
            if (b.vec) {
                const uint32_t nv = (cur.r1 - cur.r0) * vpr;
#pragma unroll
                for (int u = 0; u < PRE; ++u) {
                    const uint32_t v = u * kThreads + threadIdx.x;
                    if (v < nv) *reinterpret_cast<v8s*>(lds + cur.r0 * b.pitch + vslot[u]) = pre[u];
                }
            } else if (b.span) {
                // element e of vector v is item element l = 8v + e - lead; its row
                // and column step along with e (one division per vector)
                const uint64_t f0 = span_first(cur);
                const uint32_t lead = (uint32_t)(f0 & 7u);
                const uint32_t n = (cur.r1 - cur.r0) * g.in_w;
                const uint32_t nv = (n + lead + 7) / 8;
#pragma unroll
                for (int u = 0; u < PRE + 1; ++u) {
                    const uint32_t v = u * kThreads + threadIdx.x;
                    if (v >= nv) continue;
                    const uint32_t e0 = v == 0 ? lead : 0u;   // first element of the item in the vector
                    const uint32_t l0 = v * 8 + e0 - lead;
                    uint32_t r = fdiv(l0, b.div_w), c = l0 - r * g.in_w;
                    int16_t* row = lds + (cur.r0 + r) * b.pitch + b.cofs;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if ((uint32_t)e < e0 || v * 8 + e - lead >= n) continue;
                        row[c] = pre[u][e];
                        if (++c == g.in_w) {
                            c = 0;
                            row += b.pitch;
                        }
                    }
                }
            } else {
                const int16_t* xp = x + cur.plane * (uint64_t)g.in_h * g.in_w;
                const uint32_t n = (cur.r1 - cur.r0) * g.in_w;
                for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
                    const uint32_t r = fdiv(i, b.div_w), c = i - r * g.in_w;
                    lds[(cur.r0 + r) * b.pitch + b.cofs + c] =
                        xp[(int64_t)(cur.ih_lo + (int32_t)(cur.r0 + r)) * g.in_w + c];
                }
            }
        }
        __syncthreads();
        BandItem nb;
        const bool more = next < b.n_items;
        if (more) {
            nb = band_item(g, b, next);
            fetch(nb);                         // in flight while this item is reduced
        }

        int16_t* yp = y + cur.plane * (uint64_t)g.out_h * g.out_w;
        if constexpr (STRIP) {
            constexpr int NR = (kStrip - 1) * SH + KH;     // input rows of one strip
            const uint32_t nrows = cur.oh1 - cur.oh0;

            for (uint32_t st = my_r; my_r < rows_pp && st * kStrip < nrows; st += rows_pp) {
                const uint32_t oh_b = cur.oh0 + st * kStrip;
                // strip rows run past the tile only for outputs that are not stored;
                // the allocation has (kStrip - 1) * SH slack rows for them
                const int16_t* wrow = lds + st * kStrip * SH * b.pitch + b.cofs - g.pl;
                for (uint32_t ow = my_c; ow < g.out_w; ow += cstep) {
                    const int16_t* w0 = wrow + ow * g.sw;
                    uint32_t part[NR];
                    if constexpr (PAIR > 0) {
#pragma unroll
                        for (int rr = 0; rr < NR; ++rr)
                            part[rr] = row_window<KIND, KW>(w0 + rr * b.pitch, PAIR == 2);
                    } else {
#pragma unroll
                        for (int rr = 0; rr < NR; ++rr) {
                            Acc<KIND> a;
#pragma unroll
                            for (int kwi = 0; kwi < KW; ++kwi) a.add(w0[rr * b.pitch + kwi]);
                            part[rr] = a.v;
                        }
                    }
                    // Every row partial is read before any output is formed: the
                    // empty asm takes the values as operands, so the compiler
                    // cannot sink a read behind an output's store condition and
                    // the strip's LDS reads are all in flight together.
#pragma unroll
                    for (int rr = 0; rr < NR; ++rr) asm volatile("" : "+v"(part[rr]));
                    int16_t res[kStrip];
#pragma unroll
                    for (int o = 0; o < kStrip; ++o) {
                        const uint32_t oh = oh_b + o;
                        Acc<KIND> a;
                        a.v = part[o * SH];
#pragma unroll
                        for (int khi = 1; khi < KH; ++khi) a.merge(part[o * SH + khi]);
                        float inv = inv_full;
                        if constexpr (KIND == K_AVG) {
                            if (!g.cip) {
                                const int32_t ih0 = (int32_t)(oh * SH) - (int32_t)g.pt;
                                const int32_t iw0 = (int32_t)(ow * g.sw) - (int32_t)g.pl;
                                const uint32_t d = (uint32_t)(valid_taps(ih0, KH, 1, (int32_t)g.in_h) *
                                                              valid_taps(iw0, KW, 1, (int32_t)g.in_w));
                                inv = avg_tab ? inv_tab[d] : q88::inv_denom(d);
                            }
                        }
                        res[o] = a.finish(inv);
                    }
                    const uint32_t n_out = cur.oh1 - oh_b;   // >= 1: the strip starts inside the band
#pragma unroll
                    for (int o = 0; o < kStrip; ++o)
                        if ((uint32_t)o < n_out) yp[(uint64_t)(oh_b + o) * g.out_w + ow] = res[o];
                }
            }
        } else {
            for (uint32_t oh = cur.oh0 + my_r; my_r < rows_pp && oh < cur.oh1; oh += rows_pp) {
                // LDS row of the window's first tap: oh*sh - pt - ih_lo
                const int16_t* wrow = lds + (oh - cur.oh0) * g.sh * b.pitch + b.cofs - g.pl;
                const int32_t ih0 = (int32_t)(oh * g.sh) - (int32_t)g.pt;
                for (uint32_t ow = my_c; ow < g.out_w; ow += cstep) {
                    const int16_t* w0 = wrow + ow * g.sw;
                    Acc<KIND> a;
#pragma unroll
                    for (int32_t khi = 0; khi < (KH > 0 ? KH : ph); ++khi) {
                        const int16_t* rp = w0 + khi * dh * b.pitch;
#pragma unroll
                        for (int32_t kwi = 0; kwi < (KW > 0 ? KW : pw); ++kwi) a.add(rp[kwi * dw]);
                    }
                    float inv = inv_full;
                    if constexpr (KIND == K_AVG) {
                        if (!g.cip) {
                            const int32_t iw0 = (int32_t)(ow * g.sw) - (int32_t)g.pl;
                            const uint32_t d = (uint32_t)(valid_taps(ih0, ph, dh, (int32_t)g.in_h) *
                                                          valid_taps(iw0, pw, dw, (int32_t)g.in_w));
                            inv = avg_tab ? inv_tab[d] : q88::inv_denom(d);
                        }
                    }
                    yp[(uint64_t)oh * g.out_w + ow] = a.finish(inv);
                }
            }
        }
        if (!more) break;
        item = next;
        cur = nb;
    }
}

// ----------------------------------------------------------------- strip --
// The band layout with one strip per thread: fixed KW x KW window, row stride
// SH, 16-byte row copies, and every strip of a band (n_strips x out_w) within
// one block, so a thread owns strip threadIdx.x / out_w, column
// threadIdx.x % out_w of every item.  The next item's loads are issued into
// the registers that the current item's rows have just left, as non-temporal
// loads (each input byte is read once).  Every global access is a buffer
// access whose range is the item's own rows (input) or output band (stores),
// so loads past the item read 0 and stores past the band -- a strip's rows
// beyond the band, or a thread with no strip -- are dropped by the hardware:
// no access needs a condition, and each item issues a fixed number of loads
// and stores.  (A second item in flight per block measured slower: with the
// first items' loads competing with the second ones', the first stagings
// arrived later than the second items saved.)
template <int KIND, int KW, int SH, int PAIR>
__global__ __launch_bounds__(kThreads) void pool_strip(const int16_t* __restrict__ x,
                                                       int16_t* __restrict__ y, PoolGeom g,
                                                       BandGeom b, float inv_full) {
    touch_lines(g, b);
    extern __shared__ __align__(16) int16_t lds[];
    __shared__ float inv_tab[kInvTab];
    constexpr int KH = KW;
    constexpr int NR = (kStrip - 1) * SH + KH;   // input rows of one strip
    constexpr int PRE = kBandBytes / (kThreads * 16);
    constexpr int16_t kPadV = KIND == K_MAX ? (int16_t)-32768 : (int16_t)0;
    const bool avg_tab = KIND == K_AVG && !g.cip && (uint32_t)(KH * KW) < kInvTab;
    if (KIND == K_AVG && threadIdx.x < kInvTab) inv_tab[threadIdx.x] = q88::inv_denom(threadIdx.x);
    {
        // left / right padding columns of every row, the same for every item
        const uint32_t rcols = b.pitch - b.cofs - g.in_w;
        const uint32_t strip = b.cofs + rcols;
        if (strip) {
            const uint32_t n = b.alloc_rows * strip;
            for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
                const uint32_t r = i / strip, c = i - r * strip;
                lds[r * b.pitch + (c < b.cofs ? c : c + g.in_w)] = kPadV;
            }
        }
    }
    const uint32_t vpr = g.in_w / 8;
    uint32_t vslot[PRE];
#pragma unroll
    for (int u = 0; u < PRE; ++u) {
        const uint32_t v = u * kThreads + threadIdx.x;
        const uint32_t r = v / vpr;
        vslot[u] = r * b.pitch + b.cofs + (v - r * vpr) * 8;
    }
    const uint32_t st = threadIdx.x / g.out_w;
    const uint32_t ow = threadIdx.x - st * g.out_w;
    // LDS element of this strip's first tap, relative to the tile.  Threads with
    // no strip read the first window of row 0 (in bounds, and at the same
    // parity as every window, so the pair reads stay 4-byte aligned); their
    // stores are dropped.
    const uint32_t wofs = (st < b.n_strips ? st * kStrip * SH * b.pitch + ow * g.sw : 0u) + b.cofs - g.pl;

    // loads of an item's real input rows; an item past the end reads nothing
    auto issue = [&](uint32_t item, v8s (&pre)[PRE]) {
        const int16_t* base = x;
        uint32_t bytes = 0;
        if (item < b.n_items) {
            const BandItem it = band_item(g, b, item);
            base = x + it.plane * (uint64_t)g.in_h * g.in_w + (int64_t)(it.ih_lo + (int32_t)it.r0) * g.in_w;
            bytes = (it.r1 - it.r0) * g.in_w * 2u;
        }
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, bytes);
#pragma unroll
        for (int u = 0; u < PRE; ++u) {
            const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rs, (u * kThreads + threadIdx.x) * 16u, 0, kNonTemporal);
            pre[u] = __builtin_bit_cast(v8s, v);
        }
    };

    auto step = [&](uint32_t item, v8s (&pre)[PRE]) {
        const BandItem cur = band_item(g, b, item);
        __syncthreads();                       // the previous item's LDS reads are done
        {
            const uint32_t top = cur.r0 * b.pitch;
            const uint32_t bottom = (b.lds_rows - cur.r1) * b.pitch;
            for (uint32_t i = threadIdx.x; i < top; i += kThreads) lds[i] = kPadV;
            for (uint32_t i = threadIdx.x; i < bottom; i += kThreads) lds[cur.r1 * b.pitch + i] = kPadV;
            const uint32_t nv = (cur.r1 - cur.r0) * vpr;
#pragma unroll
            for (int u = 0; u < PRE; ++u) {
                const uint32_t v = u * kThreads + threadIdx.x;
                if (v < nv) *reinterpret_cast<v8s*>(lds + cur.r0 * b.pitch + vslot[u]) = pre[u];
            }
        }
        __syncthreads();
        issue(item + gridDim.x, pre);         // the next item, into the registers just staged

        const int16_t* w0 = lds + wofs;
        uint32_t part[NR];
        if constexpr (PAIR > 0) {
#pragma unroll
            for (int rr = 0; rr < NR; ++rr) part[rr] = row_window<KIND, KW>(w0 + rr * b.pitch, PAIR == 2);
        } else {
#pragma unroll
            for (int rr = 0; rr < NR; ++rr) {
                Acc<KIND> a;
#pragma unroll
                for (int kwi = 0; kwi < KW; ++kwi) a.add(w0[rr * b.pitch + kwi]);
                part[rr] = a.v;
            }
        }
        const __amdgpu_buffer_rsrc_t ry =
            make_rsrc(y + cur.plane * (uint64_t)g.out_h * g.out_w + (uint64_t)cur.oh0 * g.out_w,
                      (cur.oh1 - cur.oh0) * g.out_w * 2u);
#pragma unroll
        for (int o = 0; o < kStrip; ++o) {
            const uint32_t oh = cur.oh0 + st * kStrip + o;
            Acc<KIND> a;
            a.v = part[o * SH];
#pragma unroll
            for (int khi = 1; khi < KH; ++khi) a.merge(part[o * SH + khi]);
            float inv = inv_full;
            if constexpr (KIND == K_AVG) {
                if (!g.cip) {
                    const int32_t ih0 = (int32_t)(oh * SH) - (int32_t)g.pt;
                    const int32_t iw0 = (int32_t)(ow * g.sw) - (int32_t)g.pl;
                    const uint32_t d = (uint32_t)(valid_taps(ih0, KH, 1, (int32_t)g.in_h) *
                                                  valid_taps(iw0, KW, 1, (int32_t)g.in_w));
                    inv = avg_tab ? inv_tab[d] : q88::inv_denom(d);
                }
            }
            // rows past the band (and threads with no strip, st >= n_strips)
            // fall past the resource: the store is dropped
            const uint32_t off = ((st * kStrip + o) * g.out_w + ow) * 2u;
            __builtin_amdgcn_raw_buffer_store_b16(a.finish(inv), ry, off, 0, 0);
        }
    };

    uint32_t item = blockIdx.x;
    if (item >= b.n_items) return;
    v8s pre[PRE];
    issue(item, pre);
    for (;;) {
        step(item, pre);
        item += gridDim.x;
        if (item >= b.n_items) break;
    }
}

// ----------------------------------------------------------------- plane --
// Small planes (at most kPlaneMax elements): one wave per plane.  The wave
// copies its plane into a private LDS slot (16-byte loads when the planes are
// whole 16-byte vectors), then reduces the plane's output windows from LDS.
// No block barrier: a plane's whole life is one memory round trip, and a
// block holds four planes.
//
// With a fixed KW x KW window (dilation 1) the outputs split in two sets:
//   * the interior rectangle [oh_lo, oh_hi) x [ow_lo, ow_hi), whose windows
//     lie inside the plane: no bounds checks, the window origin's LDS offset
//     and the output offset advance by constants from one 64-output step to
//     the next, the taps reduce on raw values (max3 / add3);
//   * the ring of border outputs around it: pool_direct's bounds checks.
// The reduction is VALU bound at these sizes (the plane is one load round
// trip), so the interior path carries as few instructions per output as it can.
constexpr uint32_t kPlaneMax = 2048;   // elements per plane: 4 KB of LDS per wave

struct PlaneGeom {
    uint32_t oh_lo, oh_hi, ow_lo, iw_n;   // interior rows [oh_lo, oh_hi), columns [ow_lo, ow_lo + iw_n)
    uint32_t n_int, n_ring;               // interior and ring outputs
    uint32_t top_n, side, mid_n;          // ring: outputs above the interior, beside each interior
                                          // row, and beside all interior rows
    uint32_t dc;                          // 64 = (64 / iw_n) * iw_n + dc
    int32_t step_a, wrap_a;               // window origin (LDS elements): per step, per row wrap
    uint32_t step_o, wrap_o;              // output offset: per step, per row wrap
    FastDiv div_iw, div_ow, div_side;
};

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A KW x KW window entirely inside the plane, origin `w`, row pitch in_w:
// the reduction on raw values equals Acc's on shifted ones (max(x << 8) =
// max(x) << 8; sums of x << 8 mod 2^32 = (sum of x) << 8 mod 2^32, and a
// window of at most 9 taps cannot overflow int32 before the shift).
template <int KIND, int KW>
__device__ __forceinline__ int16_t window_inside(const int16_t* w, uint32_t in_w, float inv_full) {
    int32_t v[KW * KW];
    // element reads: the compiler would otherwise pair neighbours into 4-byte
    // reads, unaligned for every other window origin
    typedef __attribute__((address_space(3))) const volatile int16_t lds_i16;
    lds_i16* wv = (lds_i16*)w;
#pragma unroll
    for (int khi = 0; khi < KW; ++khi)
#pragma unroll
        for (int kwi = 0; kwi < KW; ++kwi) v[khi * KW + kwi] = wv[khi * in_w + kwi];
    if constexpr (KIND == K_MAX) {
        int32_t m = v[0];
#pragma unroll
        for (int i = 1; i < KW * KW; ++i) m = __builtin_elementwise_max(m, v[i]);
        return (int16_t)m;
    } else if constexpr (KIND == K_LP2) {
        uint32_t a = 0;
#pragma unroll
        for (int i = 0; i < KW * KW; ++i) a += (uint32_t)(v[i] * v[i]);
        return q88::lp2_finalize(a);
    } else {
        int32_t sum = 0;
#pragma unroll
        for (int i = 0; i < KW * KW; ++i) sum += KIND == K_LP1 ? __builtin_abs(v[i]) : v[i];
        const uint32_t a = (uint32_t)sum << 8;
        if constexpr (KIND == K_AVG) return q88::avg_finalize(a, inv_full);
        else return q88::acc_to_data(a);
    }
}

// One output through pool_direct's bounds checks (the ring, or any window
// when KW == 0).
template <int KIND, int KW>
__device__ __forceinline__ int16_t window_checked(const int16_t* t, const PoolGeom& g, uint32_t oh,
                                                  uint32_t ow, float inv_full) {
    const int32_t ih0 = (int32_t)(oh * g.sh) - (int32_t)g.pt;
    const int32_t iw0 = (int32_t)(ow * g.sw) - (int32_t)g.pl;
    Acc<KIND> a;
    uint32_t vh = 0;
    if constexpr (KW > 0) {
        // every tap read unconditionally at a clamped position (all KW*KW reads in
        // flight together), then masked to the pad value
        int32_t v[KW][KW];
        int32_t mw[KW];
        uint32_t iwc[KW], vw = 0;
#pragma unroll
        for (int kwi = 0; kwi < KW; ++kwi) {
            const bool ok = (uint32_t)(iw0 + kwi) < g.in_w;
            iwc[kwi] = ok ? (uint32_t)(iw0 + kwi) : 0u;
            mw[kwi] = -(int32_t)ok;
            vw += ok ? 1u : 0u;
        }
#pragma unroll
        for (int khi = 0; khi < KW; ++khi) {
            const int32_t ih = ih0 + khi;
            const bool okh = (uint32_t)ih < g.in_h;
            vh += okh ? 1u : 0u;
            const int16_t* row = t + (okh ? (uint32_t)ih : 0u) * g.in_w;
#pragma unroll
            for (int kwi = 0; kwi < KW; ++kwi) {
                // a mask, not a select: a select lets the compiler sink the read
                // into a branch and wait for each read in turn
                const int32_t m = mw[kwi] & -(int32_t)okh;
                v[khi][kwi] = ((int32_t)row[iwc[kwi]] & m) | (Acc<KIND>::kPad & ~m);
            }
        }
#pragma unroll
        for (int khi = 0; khi < KW; ++khi)
#pragma unroll
            for (int kwi = 0; kwi < KW; ++kwi) a.add(v[khi][kwi]);
        float inv = inv_full;
        if constexpr (KIND == K_AVG) {
            if (!g.cip) inv = q88::inv_denom(vh * vw);
        }
        return a.finish(inv);
    }
    for (uint32_t khi = 0; khi < g.ph; ++khi) {
        const int32_t ih = ih0 + (int32_t)(khi * g.dh);
        if ((uint32_t)ih >= g.in_h) continue;   // a padded row: skipping it is the pad's effect
        ++vh;
        const int16_t* row = t + (uint32_t)ih * g.in_w;
        for (uint32_t kwi = 0; kwi < g.pw; ++kwi) {
            const int32_t iw = iw0 + (int32_t)(kwi * g.dw);
            if ((uint32_t)iw < g.in_w) a.add(row[iw]);
        }
    }
    float inv = inv_full;
    if constexpr (KIND == K_AVG) {
        if (!g.cip)
            inv = q88::inv_denom(vh * (uint32_t)valid_taps(iw0, (int32_t)g.pw, (int32_t)g.dw, (int32_t)g.in_w));
    }
    return a.finish(inv);
}

// KW > 0: a KW x KW window with dilation 1 (interior + ring); KW == 0: any
// window, every output checked.
template <int KIND, int KW>
__global__ __launch_bounds__(kThreads) void pool_plane(const int16_t* __restrict__ x,
                                                       int16_t* __restrict__ y, PoolGeom g,
                                                       PlaneGeom p, uint64_t planes, uint32_t vec,
                                                       float inv_full) {
    __shared__ __align__(16) int16_t tile[kThreads / 64][kPlaneMax];
    touch_lines(g, p);
    const uint32_t lane = threadIdx.x & 63, w = wave_id();
    const uint64_t plane = (uint64_t)blockIdx.x * (kThreads / 64) + w;
    if (plane >= planes) return;   // the whole wave leaves; nothing waits for it
    const uint32_t hw = g.in_h * g.in_w;
    const int16_t* xp = x + plane * hw;
    int16_t* t = tile[w];
    if (vec) {
        constexpr int NV = kPlaneMax / 8 / 64;   // 16-byte vectors per lane at most
        // range-checked buffer loads (past the plane they return zero and touch no
        // memory): no branch between them, so all NV are in flight together
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(xp, hw * 2u);
        const uint32_t nv = hw / 8;
        v8s d[NV];
#pragma unroll
        for (int u = 0; u < NV; ++u)
            d[u] = __builtin_bit_cast(v8s, __builtin_amdgcn_raw_buffer_load_b128(
                                               rs, (u * 64 + lane) * 16u, 0, kNonTemporal));
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            const uint32_t v = u * 64 + lane;
            if (v < nv) *reinterpret_cast<v8s*>(t + v * 8) = d[u];
        }
    } else {
        for (uint32_t i = lane; i < hw; i += 64) t[i] = xp[i];
    }
    wave_sync();
    int16_t* yp = y + plane * (g.out_h * g.out_w);
    if constexpr (KW > 0) {
        // interior: lane's first output (r, c) of the rectangle, then +64 per step
        uint32_t r = fdiv(lane, p.div_iw);
        uint32_t c = lane - r * p.iw_n;
        int32_t a = (int32_t)(((p.oh_lo + r) * g.sh - g.pt) * g.in_w + (p.ow_lo + c) * g.sw - g.pl);
        uint32_t oo = (p.oh_lo + r) * g.out_w + p.ow_lo + c;
        for (uint32_t i = lane; i < p.n_int; i += 64) {
            yp[oo] = window_inside<KIND, KW>(t + a, g.in_w, inv_full);
            c += p.dc;
            a += p.step_a;
            oo += p.step_o;
            if (c >= p.iw_n) {
                c -= p.iw_n;
                a += p.wrap_a;
                oo += p.wrap_o;
            }
        }
        // ring: outputs above the interior, beside its rows, below it
        for (uint32_t k = lane; k < p.n_ring; k += 64) {
            uint32_t oh, ow;
            if (k < p.top_n) {
                oh = fdiv(k, p.div_ow);
                ow = k - oh * g.out_w;
            } else if (k < p.top_n + p.mid_n) {
                const uint32_t j = k - p.top_n, rr = fdiv(j, p.div_side), cc = j - rr * p.side;
                oh = p.oh_lo + rr;
                ow = cc < p.ow_lo ? cc : cc + p.iw_n;
            } else {
                const uint32_t j = k - p.top_n - p.mid_n, rr = fdiv(j, p.div_ow);
                oh = p.oh_hi + rr;
                ow = j - rr * g.out_w;
            }
            yp[oh * g.out_w + ow] = window_checked<KIND, KW>(t, g, oh, ow, inv_full);
        }
    } else {
        const uint32_t ohw = g.out_h * g.out_w;
        for (uint32_t o = lane; o < ohw; o += 64) {
            const uint32_t oh = fdiv(o, p.div_ow), ow = o - oh * g.out_w;
            yp[o] = window_checked<KIND, 0>(t, g, oh, ow, inv_full);
        }
    }
}

// Interior rectangle and ring of a plane for a KW x KW window (dilation 1);
// kw == 0: no interior (every output takes the checked path).
PlaneGeom plane_geom(const PoolGeom& g, uint32_t kw) {
    PlaneGeom p{};
    auto range = [&](uint32_t in, uint32_t out, uint32_t s, uint32_t pad, uint32_t& lo, uint32_t& hi) {
        // o is inside iff o * s >= pad and o * s - pad + kw <= in
        lo = (pad + s - 1) / s;
        const uint64_t top = (uint64_t)in + pad;
        hi = top >= kw ? (uint32_t)std::min<uint64_t>(out, (top - kw) / s + 1) : 0u;
        if (hi < lo) hi = lo;
    };
    uint32_t ow_hi = 0;
    if (kw > 0) {
        range(g.in_h, g.out_h, g.sh, g.pt, p.oh_lo, p.oh_hi);
        range(g.in_w, g.out_w, g.sw, g.pl, p.ow_lo, ow_hi);
    }
    if (kw == 0 || p.oh_hi <= p.oh_lo || ow_hi <= p.ow_lo) {
        p.oh_lo = p.oh_hi = g.out_h;   // empty interior: the "top" part of the ring is everything
        p.ow_lo = ow_hi = 0;
    }
    p.iw_n = ow_hi - p.ow_lo;
    const uint32_t ih_n = p.oh_hi - p.oh_lo;
    p.n_int = ih_n * p.iw_n;
    p.n_ring = g.out_h * g.out_w - p.n_int;
    p.top_n = p.oh_lo * g.out_w;
    p.side = g.out_w - p.iw_n;
    p.mid_n = ih_n * p.side;
    if (p.iw_n > 0) {
        const uint32_t dr = 64 / p.iw_n;
        p.dc = 64 % p.iw_n;
        p.step_a = (int32_t)(dr * g.sh * g.in_w + p.dc * g.sw);
        p.wrap_a = (int32_t)(g.sh * g.in_w) - (int32_t)(p.iw_n * g.sw);
        p.step_o = dr * g.out_w + p.dc;
        p.wrap_o = g.out_w - p.iw_n;
    }
    p.div_iw = make_fastdiv(p.iw_n);
    p.div_ow = make_fastdiv(g.out_w);
    p.div_side = make_fastdiv(p.side);
    return p;
}

// --------------------------------------------------------------- colpair --
// Planes with an even row length under a K x K window (K = 2 or 3) at stride 2
// in both directions, dilation 1 and equal top and left padding P (0 or 1):
// GW lanes per group (16 for rows of at most 32 elements, 32 for at most 64), S
// groups per plane (each taking RO consecutive output rows), 64 / GW / S planes
// per wave, no per-output addressing.  The wave copies its planes into LDS by
// 16-byte loads (per-row dword loads from memory were slower: four times the
// load instructions, each touching four partial lines), then lane j of a group
// reads input columns 2j and 2j + 1 of each row its outputs need as one dword.
// Output (oh, ow) sits on lane ow of the group holding row oh: its window covers
// input rows 2oh - P .. 2oh - P + K - 1 and input columns 2ow - P .. 2ow - P +
// K - 1, i.e. the lane's own pairs and at most one element of a neighbouring
// lane, fetched with a DPP shift (16 lanes: a row shift, whose 16-lane row is
// the group; 32 lanes: a wave shift, its value replaced at the group's edge
// lanes).  Positions outside the plane take the pad value of the reduction
// before any arithmetic (-32768 for MAX, 0 for the sums), which is the
// reference's treatment of a padded tap (PoolingKernel.cpp:151-173, 197-212).
// One plane per wave (16 lanes: S = 4; 32 lanes: S = 2) keeps many small waves
// in flight, so early waves reduce and store while later waves' loads still
// stream; with 16 lanes, S = 2 and 1 serve planes whose size keeps a single
// plane's start off 16-byte alignment.
template <int GW>
struct CpShape {
    static constexpr uint32_t kMaxHW = GW == 16 ? 1024u : 4096u;     // elements per plane
    static constexpr uint32_t kMaxOutH = GW == 16 ? 16u : 28u;       // output rows per plane
    static constexpr uint32_t kMaxIn = 2u * GW;                      // elements per input row
    static constexpr int kFront = GW;   // LDS dwords before the slots: row -1 (at most GW dwords)
};
constexpr int kDppRowShl1 = 0x101;    // lane i reads lane i + 1 of its 16-lane row
constexpr int kDppRowShr1 = 0x111;    // lane i reads lane i - 1
constexpr int kDppWaveShl1 = 0x130;   // lane i reads lane i + 1 of the wave
constexpr int kDppWaveShr1 = 0x138;   // lane i reads lane i - 1

// The value lane i + 1 (SHL) or i - 1 of the lane's GW-lane group holds; `pad`
// at the group's edge lane (j: the lane's index in its group).
template <int GW, bool SHL>
__device__ __forceinline__ int32_t dpp_neighbour(int32_t v, int32_t pad, uint32_t j) {
    if constexpr (GW == 16) {
        return __builtin_amdgcn_update_dpp(pad, v, SHL ? kDppRowShl1 : kDppRowShr1, 0xF, 0xF, false);
    } else {
        const int32_t n = __builtin_amdgcn_update_dpp(pad, v, SHL ? kDppWaveShl1 : kDppWaveShr1, 0xF, 0xF, false);
        return j == (SHL ? (uint32_t)GW - 1u : 0u) ? pad : n;
    }
}

// Taps t < K with 0 <= first + t < n.
template <int K>
__device__ __forceinline__ uint32_t taps_inside(int32_t first, uint32_t n) {
    const int32_t c = __builtin_elementwise_min(first + K, (int32_t)n) - __builtin_elementwise_max(first, 0);
    return (uint32_t)__builtin_elementwise_max(c, 0);
}

// MASK false: every window of an output inside [0, out_h) x [0, out_w) ends
// inside the plane (host-checked), so only the top padding row needs the pad
// value -- a left padding column is the DPP shift's edge value -- and rows or
// columns past the plane feed only outputs that are not stored.
template <int KIND, int K, int P, int GW, int S, bool MASK>
__global__ __launch_bounds__(kThreads) void pool_colpair(const int16_t* __restrict__ x,
                                                         int16_t* __restrict__ y, PoolGeom g,
                                                         uint64_t planes, float inv_full) {
    typedef short v2s __attribute__((ext_vector_type(2)));
    using Sh = CpShape<GW>;
    constexpr uint32_t PPW = 64u / GW / S;           // planes per wave
    constexpr uint32_t RO = (Sh::kMaxOutH + S - 1) / S;   // output rows per lane group
    constexpr int RR = 2 * ((int)RO - 1) + K;        // input rows per lane
    touch_lines(g);
    const uint32_t lane = threadIdx.x & 63, grp = lane / GW, j = lane % GW;
    const uint32_t pl = grp / S, part = grp % S;      // plane in the wave, row part
    const uint64_t plane0 = ((uint64_t)blockIdx.x * (kThreads / 64) + wave_id()) * PPW;
    if (plane0 >= planes) return;   // the whole wave leaves
    const uint32_t np = (uint32_t)(planes - plane0 < PPW ? planes - plane0 : PPW);
    const uint32_t hw = g.in_h * g.in_w, ohw = g.out_h * g.out_w;
    // the wave's planes (contiguous, 16-byte aligned) are copied into its LDS slot
    // by 16-byte range-checked loads (past the planes they read 0); every store is
    // range-checked against the wave's planes
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + plane0 * hw, np * hw * 2u);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(y + plane0 * ohw, np * ohw * 2u);
    constexpr int SLOT = PPW * Sh::kMaxHW / 2;      // LDS dwords per wave
    // row reads reach, from a slot's start, the last plane's row 2 RO S + K - 3
    // (at most GW dwords each) and its column pair: past the last slot, slack
    constexpr int REACH = ((int)PPW - 1) * (int)Sh::kMaxHW / 2 + (2 * (int)(RO * S) + K - 3) * GW + GW;
    constexpr int BACK = REACH > SLOT ? REACH - SLOT : 0;
    __shared__ __align__(16) uint32_t tile[Sh::kFront + kThreads / 64 * SLOT + BACK];
    uint32_t* t = tile + Sh::kFront + wave_id() * SLOT;
    {
        constexpr int NV = SLOT / 4 / 64;   // 16-byte vectors per lane
        v4u v[NV];
#pragma unroll
        for (int u = 0; u < NV; ++u)
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, (u * 64 + lane) * 16u, 0, kNonTemporal);
#pragma unroll
        for (int u = 0; u < NV; ++u) *reinterpret_cast<v4u*>(t + (u * 64 + lane) * 4) = v[u];
    }
    wave_sync();
    // register row i holds input row r0 + i; rows outside the plane read what
    // lies there (inside the slots or their slack) and are masked to the pad
    // value through a bit mask, not a select: a select let the compiler sink a
    // read into a branch, after which the first row waited for every read
    const int32_t r0 = (int32_t)(2 * RO * part) - P;
    const uint32_t pitch = g.in_w / 2;
    const uint32_t* tl = t + (int32_t)(pl * (hw / 2) + j) + r0 * (int32_t)pitch;
    constexpr uint32_t kPadPair = KIND == K_MAX ? 0x80008000u : 0u;
    const uint32_t col_m = 2u * j < g.in_w ? ~0u : 0u;
    uint32_t d[RR];
    typedef __attribute__((address_space(3))) const uint32_t lds_u32;
    lds_u32* lp = (lds_u32*)tl;   // 32-bit LDS address: one add per row
#pragma unroll
    for (int i = 0; i < RR; ++i, lp += pitch) {
        uint32_t m;
        if constexpr (MASK) m = (uint32_t)(r0 + i) < g.in_h ? col_m : 0u;
        else m = i < P && part == 0 ? 0u : ~0u;   // only the top padding row
        d[i] = (*lp & m) | (kPadPair & ~m);
    }
    // output offsets: the lane's first row and column (past the range when the
    // column is outside the plane), then one row step per output
    const uint32_t oh0 = RO * part;
    const uint32_t yb = j < g.out_w ? (pl * ohw + oh0 * g.out_w + j) * 2u : kOob;
    // the outputs; CIP: AVG with count_include_pad (one denominator), a uniform
    // choice made once
    auto emit = [&](auto cip_tag) {
        constexpr bool CIP = decltype(cip_tag)::value;
        // AVG without count_include_pad: inv * 2^-8 (avg_finalize8) for each count
        // of window rows inside the plane (0..K) times this lane's columns inside
        // it, computed once (no division per output)
        float inv8[K + 1];
        if constexpr (KIND == K_AVG && !CIP) {
            const uint32_t vcols = taps_inside<K>(2 * (int32_t)j - P, g.in_w);
#pragma unroll
            for (int vr = 0; vr <= K; ++vr)
                inv8[vr] = q88::mul_rn(q88::inv_denom((uint32_t)vr * vcols), 1.0f / 256.0f);
        }
        const float inv8_full = q88::mul_rn(inv_full, 1.0f / 256.0f);
#pragma unroll
        for (uint32_t o = 0; o < RO; ++o) {
            const uint32_t* r = d + 2 * o;
            int32_t out;
            if constexpr (KIND == K_MAX) {
                // rows by the packed 16-bit max, then the columns of the low halves
                v2s m = __builtin_elementwise_max(__builtin_bit_cast(v2s, r[0]), __builtin_bit_cast(v2s, r[1]));
                if constexpr (K == 3) m = __builtin_elementwise_max(m, __builtin_bit_cast(v2s, r[2]));
                const int32_t e0 = m[0], e1 = m[1];
                int32_t v = __builtin_elementwise_max(e0, e1);
                if constexpr (P == 0 && K == 3) v = __builtin_elementwise_max(v, dpp_neighbour<GW, true>(e0, -32768, j));
                if constexpr (P == 1 && K == 2) v = e0;
                if constexpr (P == 1) v = __builtin_elementwise_max(v, dpp_neighbour<GW, false>(e1, -32768, j));
                out = v;
            } else {
                uint32_t s;
                if constexpr (P == 0 && K == 2 && KIND != K_LP1) {
                    // the window is the lane's own pairs of two rows: sums of x or
                    // x^2 by v_dot2 (the int32 sum wraps like the reference accumulator)
                    const v2s r0v = __builtin_bit_cast(v2s, r[0]), r1v = __builtin_bit_cast(v2s, r[1]);
                    const v2s w0 = KIND == K_LP2 ? r0v : v2s{1, 1}, w1 = KIND == K_LP2 ? r1v : v2s{1, 1};
                    s = (uint32_t)__builtin_amdgcn_sdot2(r1v, w1, __builtin_amdgcn_sdot2(r0v, w0, 0, false), false);
                } else {
                    // each column's rows summed (x, |x| or x^2, as wrapping uint32)
                    auto term = [](int32_t e) -> uint32_t {
                        if constexpr (KIND == K_LP1) return (uint32_t)__builtin_abs(e);
                        else if constexpr (KIND == K_LP2) return (uint32_t)(e * e);
                        else return (uint32_t)e;
                    };
                    uint32_t c0 = 0, c1 = 0;
#pragma unroll
                    for (int tp = 0; tp < K; ++tp) {
                        c0 += term((int32_t)(int16_t)(r[tp] & 0xFFFFu));
                        c1 += term((int32_t)r[tp] >> 16);
                    }
                    if constexpr (P == 0 && K == 3) s = c0 + c1 + (uint32_t)dpp_neighbour<GW, true>((int32_t)c0, 0, j);
                    else if constexpr (P == 0) s = c0 + c1;
                    else if constexpr (K == 3) s = c0 + c1 + (uint32_t)dpp_neighbour<GW, false>((int32_t)c1, 0, j);
                    else s = c0 + (uint32_t)dpp_neighbour<GW, false>((int32_t)c1, 0, j);
                }
                if constexpr (KIND == K_AVG) {
                    float inv = inv8_full;
                    if constexpr (!CIP) {
                        const uint32_t vr = taps_inside<K>(r0 + 2 * (int32_t)o, g.in_h);
                        inv = inv8[0];
#pragma unroll
                        for (int tp = 1; tp <= K; ++tp) inv = vr == (uint32_t)tp ? inv8[tp] : inv;
                    }
                    out = q88::avg_finalize8(s << 8, inv);
                } else if constexpr (KIND == K_LP2) {
                    out = q88::lp2_finalize(s);
                } else {
                    out = q88::acc_to_data(s << 8);
                }
            }
            // (kOob plus a row offset stays below 2^32: still past the range)
            const uint32_t yo = oh0 + o < g.out_h ? yb + o * g.out_w * 2u : kOob;
            __builtin_amdgcn_raw_buffer_store_b16((int16_t)out, ry, yo, 0, 0);
        }
    };
    if (KIND == K_AVG && !g.cip) emit(std::false_type{});
    else emit(std::true_type{});
}

// ---------------------------------------------------------------- direct --
template <int KIND>
__global__ __launch_bounds__(kThreads) void pool_direct(const int16_t* __restrict__ x,
                                                        int16_t* __restrict__ y, PoolGeom g,
                                                        uint64_t total, float inv_full) {
    touch_lines(g);
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    const uint64_t ohw = (uint64_t)g.out_h * g.out_w;
    for (uint64_t o = (uint64_t)blockIdx.x * kThreads + threadIdx.x; o < total; o += stride) {
        const uint64_t plane = o / ohw;
        const uint32_t rem = (uint32_t)(o - plane * ohw);
        const uint32_t oh = rem / g.out_w, ow = rem - (rem / g.out_w) * g.out_w;
        const int16_t* xp = x + plane * (uint64_t)g.in_h * g.in_w;
        const int64_t ih0 = (int64_t)oh * g.sh - g.pt;
        const int64_t iw0 = (int64_t)ow * g.sw - g.pl;
        Acc<KIND> a;
        uint32_t vh = 0, vw = 0;
        for (uint32_t khi = 0; khi < g.ph; ++khi) {
            const int64_t ih = ih0 + (int64_t)khi * g.dh;
            if (ih < 0 || ih >= (int64_t)g.in_h) continue;
            ++vh;
            for (uint32_t kwi = 0; kwi < g.pw; ++kwi) {
                const int64_t iw = iw0 + (int64_t)kwi * g.dw;
                if (iw >= 0 && iw < (int64_t)g.in_w) a.add(xp[(uint64_t)ih * g.in_w + iw]);
            }
        }
        float inv = inv_full;
        if constexpr (KIND == K_AVG) {
            if (!g.cip) {
                for (uint32_t t = 0; t < g.pw; ++t) {
                    const int64_t p = iw0 + (int64_t)t * g.dw;
                    vw += (p >= 0 && p < (int64_t)g.in_w) ? 1u : 0u;
                }
                inv = q88::inv_denom(vh * vw);
            }
        }
        y[o] = a.finish(inv);
    }
}

// Input rows needed by `bh` consecutive output rows.
uint64_t rows_needed(const PoolGeom& g, uint32_t bh) {
    return (uint64_t)(bh - 1) * g.sh + (uint64_t)(g.ph - 1) * g.dh + 1;
}

// Blocks of kThreads threads with `lds` dynamic LDS bytes resident on the whole
// device at once (occupancy, at most max_per_cu, x CU count), kPoolBlocks if
// the runtime cannot say.
uint64_t resident_blocks(const void* kernel, uint32_t lds, int max_per_cu) {
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        per_cu <= 0 || cus <= 0) {
        (void)hipGetLastError();
        return kPoolBlocks;
    }
    return (uint64_t)(per_cu < max_per_cu ? per_cu : max_per_cu) * (uint64_t)cus;
}

// 1.0f / (float)d on the host: IEEE round-to-nearest-even, like the device path.
float host_inv_denom(uint64_t d) { return d ? 1.0f / (float)d : 0.0f; }

template <int KIND>
int pool_launch(const int16_t* x, int16_t* y, uint64_t planes, const PoolGeom& g, hipStream_t s) {
    const uint64_t full = (uint64_t)g.ph * g.pw;   // count_include_pad denominator
    const float inv_full = host_inv_denom(full > 0xFFFFFFFFull ? 0 : full);
    const uint64_t total = planes * g.out_h * g.out_w;
    if (g.ph == 0 || g.pw == 0 || g.in_h == 0 || g.in_w == 0) {
        // empty window or input: every output is the finaliser of the initial accumulator
        hipLaunchKernelGGL(pool_direct<KIND>, dim3((uint32_t)cm_grid_blocks(total, kThreads)),
                           dim3(kThreads), 0, s, x, y, g, total, inv_full);
        return cm_check_launch("pool_direct");
    }
    const bool global = g.out_h == 1 && g.out_w == 1 && g.ph == g.in_h && g.pw == g.in_w &&
                        g.pt == 0 && g.pl == 0 && g.dh == 1 && g.dw == 1;
    if (global) {
        const uint64_t hw = (uint64_t)g.in_h * g.in_w;
        if (hw > 0xFFFFFFFFull) return cm_set_error(CM_ERR_RANGE, "pool: plane too large");
        const uint32_t vec_ok = (hw % 8 == 0) && (((uintptr_t)x & 15u) == 0);
        const uint64_t blocks = (planes + 3) / 4;
        if (blocks > 0x7FFFFFFFull) return cm_set_error(CM_ERR_RANGE, "pool: too many planes");
        // no padding: the valid count equals the window size for either cip; the
        // loads per lane in flight fitted to the plane's 16-byte vectors
        const uint64_t per_lane = (hw / 8 + 63) / 64;
        const float inv_hw = host_inv_denom(hw);
        if (hw <= 128) {   // small planes: sixteen lanes each
            const dim3 grid((uint32_t)((planes + 15) / 16)), block(kThreads);
            if ((planes + 15) / 16 > 0x7FFFFFFFull) return cm_set_error(CM_ERR_RANGE, "pool: too many planes");
            if (hw <= 16) hipLaunchKernelGGL((pool_gsmall<KIND, 1>), grid, block, 0, s, x, y, planes, (uint32_t)hw, inv_hw);
            else if (hw <= 32) hipLaunchKernelGGL((pool_gsmall<KIND, 2>), grid, block, 0, s, x, y, planes, (uint32_t)hw, inv_hw);
            else if (hw <= 64) hipLaunchKernelGGL((pool_gsmall<KIND, 4>), grid, block, 0, s, x, y, planes, (uint32_t)hw, inv_hw);
            else hipLaunchKernelGGL((pool_gsmall<KIND, 8>), grid, block, 0, s, x, y, planes, (uint32_t)hw, inv_hw);
            return cm_check_launch("pool_gsmall");
        }
#define CM_POOL_GLOBAL(NB)                                                                       \
    hipLaunchKernelGGL((pool_global<KIND, NB>), dim3((uint32_t)blocks), dim3(kThreads), 0, s, x, y, \
                       planes, (uint32_t)hw, inv_hw, vec_ok)
        if (per_lane <= 1) CM_POOL_GLOBAL(1);
        else if (per_lane <= 2) CM_POOL_GLOBAL(2);
        else if (per_lane <= 4) CM_POOL_GLOBAL(4);
        else CM_POOL_GLOBAL(8);
#undef CM_POOL_GLOBAL
        return cm_check_launch("pool_global");
    }
    // The band kernel indexes with 32-bit arithmetic: only shapes well inside
    // that range take it.  Band height: as many output rows as fit the LDS
    // budget (+16 B alignment slack).
    const bool small = g.in_h < (1u << 20) && g.in_w < (1u << 20) && g.sh < (1u << 10) &&
                       g.sw < (1u << 10) && g.dh < (1u << 10) && g.dw < (1u << 10) &&
                       g.pt < (1u << 20) && g.pl < (1u << 20) && g.ph < (1u << 10) &&
                       g.pw < (1u << 10) && (uint64_t)g.out_w * g.sw < (1u << 30) &&
                       (uint64_t)g.out_h * g.sh < (1u << 30) &&
                       (uint64_t)g.in_h * g.in_w < (1u << 30);
    // planes under a 2x2 / 3x3 window at stride 2 with even rows of at most 32
    // elements (16-lane groups) or 64 (32-lane groups, one plane per wave): rows
    // in registers (pool_colpair)
    const uint32_t kcp = g.ph == g.pw && (g.ph == 2 || g.ph == 3) ? g.ph : 0;
    const uint64_t hw = (uint64_t)g.in_h * g.in_w;
    const bool cp_geom = kcp && g.sh == 2 && g.sw == 2 && g.dh == 1 && g.dw == 1 && g.pt == g.pl &&
                         g.pt <= 1 && g.in_w % 2 == 0 && ((uintptr_t)x & 15u) == 0;
    const bool cp16 = cp_geom && g.in_w <= CpShape<16>::kMaxIn && hw <= CpShape<16>::kMaxHW &&
                      g.out_h <= CpShape<16>::kMaxOutH && g.out_w <= 16u;
    const bool cp32 = !cp16 && cp_geom && hw % 8 == 0 && g.in_w <= CpShape<32>::kMaxIn &&
                      hw <= CpShape<32>::kMaxHW && g.out_h <= CpShape<32>::kMaxOutH && g.out_w <= 32u;
    if ((cp16 || cp32) && (planes + 3) / 4 <= 0x7FFFFFFFull) {
        // 16 lanes: one plane per wave when a plane's start stays 16-byte aligned,
        // else two or four
        const uint32_t S = cp32 ? 2u : hw % 8 == 0 ? 4u : (hw % 4 == 0 ? 2u : 1u);
        const uint64_t per_block = 4 * (64 / (cp32 ? 32 : 16) / S);
        const dim3 grid((uint32_t)((planes + per_block - 1) / per_block)), block(kThreads);
        // windows of the last output row / column end inside the plane: no masks
        const bool inside = 2ull * (g.out_h - 1) + kcp - 1 < (uint64_t)g.in_h + g.pt &&
                            2ull * (g.out_w - 1) + kcp - 1 < (uint64_t)g.in_w + g.pl;
#define CM_COLPAIR_M(K_, P_, GW_, S_) \
    do { if (inside) hipLaunchKernelGGL((pool_colpair<KIND, K_, P_, GW_, S_, false>), grid, block, 0, s, x, y, g, planes, inv_full); \
         else hipLaunchKernelGGL((pool_colpair<KIND, K_, P_, GW_, S_, true>), grid, block, 0, s, x, y, g, planes, inv_full); } while (0)
#define CM_COLPAIR_S(K_, P_) \
    do { if (cp32) CM_COLPAIR_M(K_, P_, 32, 2); \
         else if (S == 4) CM_COLPAIR_M(K_, P_, 16, 4); else if (S == 2) CM_COLPAIR_M(K_, P_, 16, 2); \
         else CM_COLPAIR_M(K_, P_, 16, 1); } while (0)
        if (kcp == 3) {
            if (g.pt) CM_COLPAIR_S(3, 1); else CM_COLPAIR_S(3, 0);
        } else {
            if (g.pt) CM_COLPAIR_S(2, 1); else CM_COLPAIR_S(2, 0);
        }
#undef CM_COLPAIR_S
#undef CM_COLPAIR_M
        return cm_check_launch("pool_colpair");
    }
    // small planes: one wave per plane, the plane in LDS
    if (small && (uint64_t)g.in_h * g.in_w <= kPlaneMax && (uint64_t)g.out_h * g.out_w <= (1u << 24)) {
        const uint64_t blocks = (planes + 3) / 4;
        if (blocks <= 0x7FFFFFFFull) {
            const uint32_t vec = ((uint64_t)g.in_h * g.in_w) % 8 == 0 && (((uintptr_t)x & 15u) == 0);
            const uint32_t kwp = g.dh == 1 && g.dw == 1 && g.ph == g.pw && (g.ph == 2 || g.ph == 3) ? g.ph : 0;
            const PlaneGeom pg = plane_geom(g, kwp);
            if (kwp == 3)
                hipLaunchKernelGGL((pool_plane<KIND, 3>), dim3((uint32_t)blocks), dim3(kThreads), 0, s, x, y,
                                   g, pg, planes, vec, inv_full);
            else if (kwp == 2)
                hipLaunchKernelGGL((pool_plane<KIND, 2>), dim3((uint32_t)blocks), dim3(kThreads), 0, s, x, y,
                                   g, pg, planes, vec, inv_full);
            else
                hipLaunchKernelGGL((pool_plane<KIND, 0>), dim3((uint32_t)blocks), dim3(kThreads), 0, s, x, y,
                                   g, pg, planes, vec, inv_full);
            return cm_check_launch("pool_plane");
        }
    }
    // Padded LDS tile: columns [-pl, in_w + pr) at offset cofs = round_up(pl, 8),
    // pitch a multiple of 8; rows = the window footprint of `band_h` output rows.
    const uint64_t pr_need = (uint64_t)(g.out_w - 1) * g.sw + (uint64_t)(g.pw - 1) * g.dw + 1;
    const uint64_t cofs = ((uint64_t)g.pl + 7) / 8 * 8;
    const uint64_t right = pr_need > (uint64_t)g.pl + g.in_w ? pr_need - g.pl : g.in_w;
    const uint64_t pitch = (cofs + right + 7) / 8 * 8;
    uint32_t band_h = 0;
    if (small && rows_needed(g, 1) * pitch * 2 <= kBandBytes) {
        uint32_t lo = 1, hi = g.out_h;
        while (lo < hi) {
            const uint32_t mid = lo + (hi - lo + 1) / 2;
            if (rows_needed(g, mid) * pitch * 2 <= kBandTarget) lo = mid; else hi = mid - 1;
        }
        band_h = lo;
    }
    const bool unit_dil = g.dh == 1 && g.dw == 1;
    const uint32_t kwin = unit_dil && g.ph == g.pw && (g.ph == 2 || g.ph == 3) ? g.ph : 0;
    const uint32_t sh = kwin && (g.sh == 1 || g.sh == 2) ? g.sh : 0;
    const uint32_t vec = (g.in_w % 8 == 0) && (((uintptr_t)x & 15u) == 0);
    // pool_strip: fixed window and row stride, 16-byte rows, and every strip of
    // a band in one block (bands of at most kThreads / out_w strips)
    const bool one_pass = band_h > 0 && sh && vec && g.out_w <= (uint32_t)kThreads;
    if (one_pass) band_h = std::min<uint32_t>(band_h, (kThreads / g.out_w) * kStrip);
    if (band_h > 0) {
        const uint32_t n_bands = (g.out_h + band_h - 1) / band_h;
        const uint64_t items = planes * n_bands;
        if (items <= 0x7FFFFFFFull) {
            BandGeom b;
            b.band_h = band_h;
            b.n_bands = n_bands;
            b.n_items = (uint32_t)items;
            b.pitch = (uint32_t)pitch;
            b.cofs = (uint32_t)cofs;
            b.lds_rows = (uint32_t)rows_needed(g, band_h);
            b.vec = vec;
            {
                // the range rounds up to 16 bytes: buffer loads check it per dword,
                // and the last element may share a dword with bytes past x (the
                // 16-byte chunk holding x's last byte lies in x's page, x being
                // 16-byte aligned)
                const uint64_t xb = ((uint64_t)g.in_h * g.in_w * 2 * planes + 15) & ~15ull;
                b.span = !vec && ((uintptr_t)x & 15u) == 0 && xb < 0x80000000ull;
                b.x_bytes = b.span ? (uint32_t)xb : 0u;
            }
            b.n_strips = (band_h + kStrip - 1) / kStrip;
            b.div_w = make_fastdiv(g.in_w);
            b.alloc_rows = b.lds_rows + (sh ? (kStrip - 1) * sh : 0);
            // + 16 B: a 2-wide window at an odd column reads its taps as the
            // aligned pair that starts one element later
            const uint32_t lds = b.alloc_rows * b.pitch * 2 + 16;
            // strip path with an even column stride: every window starts at the
            // same parity, so its taps are read as aligned pairs (PAIR 1: the
            // window starts 4-byte aligned, 2: one element past that)
            const int pair = sh && g.sw % 2 == 0 ? ((b.cofs - g.pl) % 2 == 0 ? 1 : 2) : 0;
            // persistent blocks: at most as many as are resident at once (a block
            // beyond that would start a second round and double the tail)
#define CM_LAUNCH(KERNEL)                                                                      \
    do {                                                                                       \
        const uint64_t cap = resident_blocks((const void*)KERNEL, lds, kPersistPerCu);          \
        const dim3 grid((uint32_t)(items < cap ? items : cap)), block(kThreads);               \
        hipLaunchKernelGGL(KERNEL, grid, block, lds, s, x, y, g, b, inv_full);                 \
    } while (0)
#define CM_BAND(KW_, SH_, P_) CM_LAUNCH((pool_band<KIND, KW_, KW_, SH_, P_>))
#define CM_BAND_P(KW_, SH_) \
    do { if (pair == 1) CM_BAND(KW_, SH_, 1); else if (pair == 2) CM_BAND(KW_, SH_, 2); else CM_BAND(KW_, SH_, 0); } while (0)
#define CM_STRIP(KW_, SH_, P_) CM_LAUNCH((pool_strip<KIND, KW_, SH_, P_>))
#define CM_STRIP_P(KW_, SH_) \
    do { if (pair == 1) CM_STRIP(KW_, SH_, 1); else if (pair == 2) CM_STRIP(KW_, SH_, 2); else CM_STRIP(KW_, SH_, 0); } while (0)
            if (one_pass) {
                if (kwin == 3) {
                    if (sh == 2) CM_STRIP_P(3, 2); else CM_STRIP_P(3, 1);
                } else {
                    if (sh == 2) CM_STRIP_P(2, 2); else CM_STRIP_P(2, 1);
                }
                return cm_check_launch("pool_strip");
            }
            if (kwin == 3) {
                if (sh == 2) CM_BAND_P(3, 2); else if (sh == 1) CM_BAND_P(3, 1); else CM_BAND(3, 0, 0);
            } else if (kwin == 2) {
                if (sh == 2) CM_BAND_P(2, 2); else if (sh == 1) CM_BAND_P(2, 1); else CM_BAND(2, 0, 0);
            } else {
                CM_BAND(0, 0, 0);
            }
#undef CM_STRIP_P
#undef CM_STRIP
#undef CM_BAND_P
#undef CM_BAND
#undef CM_LAUNCH
            return cm_check_launch("pool_band");
        }
    }
    hipLaunchKernelGGL(pool_direct<KIND>, dim3((uint32_t)cm_grid_blocks(total, kThreads)),
                       dim3(kThreads), 0, s, x, y, g, total, inv_full);
    return cm_check_launch("pool_direct");
}

// Exhaustive finaliser sweep: mode 0 = LP p=2 over accumulators lo + i;
// mode 1 = AVG over accumulators (lo + i) << 8 with denominator d.
// checksum += (uint16)out * ((lo + i) | 1), modulo 2^64.
__global__ __launch_bounds__(kThreads) void pool_finalize_sweep(uint32_t mode, uint32_t lo,
                                                                uint32_t count, uint32_t d,
                                                                unsigned long long* checksum) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    unsigned long long s = 0;
    const float inv = q88::inv_denom(d);
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < count; i += stride) {
        const uint32_t v = lo + (uint32_t)i;
        const int16_t out = mode == 0 ? q88::lp2_finalize(v) : q88::avg_finalize(v << 8, inv);
        s += (unsigned long long)(uint16_t)out * (unsigned long long)(v | 1u);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) atomicAdd(checksum, s);
}

}  // namespace

int cm_pool_launch(const int16_t* x, int16_t* y, uint32_t batch, uint32_t ch, uint32_t in_h,
                   uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t ph, uint32_t pw,
                   uint32_t sh, uint32_t sw, uint32_t pad_top, uint32_t pad_left, uint32_t dh,
                   uint32_t dw, uint32_t pool_type, uint32_t lp_order, uint32_t cip,
                   hipStream_t s) {
    const uint64_t planes = (uint64_t)batch * ch;
    if (planes == 0 || out_h == 0 || out_w == 0) return CM_OK;
    const PoolGeom g{in_h, in_w, out_h, out_w, ph, pw, sh, sw, pad_top, pad_left, dh, dw,
                     pool_type, lp_order, cip};
    // pool_type 0 MAX, 1 AVG, anything else Lp; lp_order 1 -> p=1, else p=2
    // (PoolingKernel.cpp:214-224, 261-263)
    if (pool_type == CM_POOL_MAX) return pool_launch<K_MAX>(x, y, planes, g, s);
    if (pool_type == CM_POOL_AVG) return pool_launch<K_AVG>(x, y, planes, g, s);
    if (lp_order == 1u) return pool_launch<K_LP1>(x, y, planes, g, s);
    return pool_launch<K_LP2>(x, y, planes, g, s);
}

int cm_finalize_sweep_launch(uint32_t mode, uint32_t lo, uint32_t count, uint32_t d,
                             unsigned long long* checksum, hipStream_t s) {
    hipLaunchKernelGGL(pool_finalize_sweep, dim3((uint32_t)cm_grid_blocks(count, kThreads, 4096)),
                       dim3(kThreads), 0, s, mode, lo, count, d, checksum);
    return cm_check_launch("pool_finalize_sweep");
}
