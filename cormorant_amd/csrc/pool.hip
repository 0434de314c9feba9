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
//     16-byte loads, cross-lane reduction;
//   * band:   a block stages the input rows that a band of output rows needs
//     in LDS (16-byte loads), then computes the band from LDS;
//   * direct: rows too wide for LDS -- each thread reads its window from HBM.
#include "cm_internal.h"
#include "q88.h"

namespace {

typedef short v8s __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr uint32_t kLdsBytes = 32768;

struct PoolGeom {
    uint32_t in_h, in_w, out_h, out_w, ph, pw, sh, sw, pt, pl, dh, dw;
    uint32_t pool_type, lp_order, cip;
};

// Accumulator state for one output: uint32 wrap sums, int32 max.
struct PoolAcc {
    uint32_t acc;
    __device__ __forceinline__ void init(uint32_t type) { acc = type == CM_POOL_MAX ? 0x80000000u : 0u; }
    __device__ __forceinline__ void add(uint32_t type, uint32_t lp, int32_t x) {
        if (type == CM_POOL_MAX) {
            const int32_t v = x << 8;
            acc = (uint32_t)__builtin_elementwise_max((int32_t)acc, v);
        } else if (type == CM_POOL_AVG) {
            acc += (uint32_t)x << 8;
        } else if (lp == 1u) {
            acc += (uint32_t)__builtin_abs(x) << 8;
        } else {
            acc += (uint32_t)(x * x);
        }
    }
};

__device__ __forceinline__ int16_t pool_finish(uint32_t type, uint32_t lp, uint32_t acc,
                                               uint32_t denom) {
    if (type == CM_POOL_MAX) return q88::acc_to_data(acc);
    if (type == CM_POOL_AVG) return q88::avg_finalize(acc, q88::inv_denom(denom));
    if (lp == 1u) return q88::acc_to_data(acc);
    return q88::lp2_finalize(acc);
}

// Number of window taps t < k with 0 <= base + t*d < lim.
__device__ __forceinline__ uint32_t valid_taps(int64_t base, uint32_t k, uint32_t d, uint32_t lim) {
    uint32_t n = 0;
    for (uint32_t t = 0; t < k; ++t) {
        const int64_t p = base + (int64_t)t * d;
        n += (p >= 0 && p < (int64_t)lim) ? 1u : 0u;
    }
    return n;
}

// ---------------------------------------------------------------- global --
// One wavefront reduces one plane of `hw` elements.
__global__ __launch_bounds__(kThreads) void pool_global(const int16_t* __restrict__ x,
                                                        int16_t* __restrict__ y, uint64_t planes,
                                                        uint32_t hw, uint32_t type, uint32_t lp,
                                                        uint32_t denom, uint32_t vec_ok) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t plane = (uint64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (plane >= planes) return;
    const int16_t* xp = x + plane * hw;
    PoolAcc a;
    a.init(type);
    uint32_t done = 0;
    if (vec_ok) {
        const v8s* xv = reinterpret_cast<const v8s*>(xp);
        const uint32_t nv = hw / 8;
        for (uint32_t v = lane; v < nv; v += 64) {
            const v8s t = __builtin_nontemporal_load(xv + v);
#pragma unroll
            for (int j = 0; j < 8; ++j) a.add(type, lp, t[j]);
        }
        done = nv * 8;
    }
    for (uint32_t i = done + lane; i < hw; i += 64) a.add(type, lp, xp[i]);
    // cross-lane reduction: max for MAX, wrapping add otherwise
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)a.acc, off, 64);
        a.acc = type == CM_POOL_MAX ? (uint32_t)__builtin_elementwise_max((int32_t)a.acc, (int32_t)o)
                                    : a.acc + o;
    }
    if (lane == 0) y[plane] = pool_finish(type, lp, a.acc, denom);
}

// ------------------------------------------------------------------ band --
// Block = (plane, band of `band_h` output rows).  Stages input rows
// [r_lo, r_hi) (full width) in LDS, then each thread produces outputs.
__global__ __launch_bounds__(kThreads) void pool_band(const int16_t* __restrict__ x,
                                                      int16_t* __restrict__ y, PoolGeom g,
                                                      uint32_t band_h, uint32_t n_bands) {
    extern __shared__ __align__(16) int16_t lds[];
    const uint64_t plane = blockIdx.x / n_bands;
    const uint32_t band = blockIdx.x - (uint32_t)(plane * n_bands);
    const uint32_t oh0 = band * band_h;
    const uint32_t oh1 = min(oh0 + band_h, g.out_h);

    // input rows touched by output rows [oh0, oh1)
    const int64_t lo = (int64_t)oh0 * g.sh - g.pt;
    const int64_t hi = (int64_t)(oh1 - 1) * g.sh - g.pt + (int64_t)(g.ph - 1) * g.dh + 1;
    const int64_t r_lo = lo < 0 ? 0 : lo;
    const int64_t r_hi = hi > (int64_t)g.in_h ? (int64_t)g.in_h : hi;
    const uint64_t plane_elems = (uint64_t)g.in_h * g.in_w;
    const int16_t* xp = x + plane * plane_elems;

    if (r_hi > r_lo) {
        // copy elements [e0, e1) of the plane to lds[shift + (e - e0)], where
        // shift aligns the 16-byte body of the copy in LDS with global memory.
        const uint64_t e0 = (uint64_t)r_lo * g.in_w, e1 = (uint64_t)r_hi * g.in_w;
        const int16_t* src = xp + e0;
        const uint32_t shift = (uint32_t)(((uintptr_t)src >> 1) & 7u);
        const uint32_t n = (uint32_t)(e1 - e0);
        const uint32_t head = min((8u - shift) & 7u, n);
        const uint32_t nv = (n - head) / 8;
        const uint32_t body_end = head + nv * 8;
        int16_t* dst = lds + shift;
        if (threadIdx.x < head) dst[threadIdx.x] = src[threadIdx.x];
        const v8s* sv = reinterpret_cast<const v8s*>(src + head);
        v8s* dv = reinterpret_cast<v8s*>(dst + head);
        for (uint32_t v = threadIdx.x; v < nv; v += kThreads) dv[v] = __builtin_nontemporal_load(sv + v);
        for (uint32_t i = body_end + threadIdx.x; i < n; i += kThreads) dst[i] = src[i];
    }
    __syncthreads();

    const int16_t* rows = lds + (uint32_t)(((uintptr_t)(xp + (uint64_t)r_lo * g.in_w) >> 1) & 7u);
    const uint32_t count = (oh1 - oh0) * g.out_w;
    int16_t* yp = y + plane * (uint64_t)g.out_h * g.out_w + (uint64_t)oh0 * g.out_w;
    const int16_t pad = g.pool_type == CM_POOL_MAX ? (int16_t)-32768 : (int16_t)0;
    for (uint32_t idx = threadIdx.x; idx < count; idx += kThreads) {
        const uint32_t r = idx / g.out_w;
        const uint32_t ow = idx - r * g.out_w;
        const int64_t ih0 = (int64_t)(oh0 + r) * g.sh - g.pt;
        const int64_t iw0 = (int64_t)ow * g.sw - g.pl;
        PoolAcc a;
        a.init(g.pool_type);
        for (uint32_t khi = 0; khi < g.ph; ++khi) {
            const int64_t ih = ih0 + (int64_t)khi * g.dh;
            const bool ih_ok = ih >= 0 && ih < (int64_t)g.in_h;
            const int16_t* row = rows + (ih_ok ? (uint64_t)(ih - r_lo) * g.in_w : 0);
            for (uint32_t kwi = 0; kwi < g.pw; ++kwi) {
                const int64_t iw = iw0 + (int64_t)kwi * g.dw;
                const bool ok = ih_ok && iw >= 0 && iw < (int64_t)g.in_w;
                a.add(g.pool_type, g.lp_order, ok ? row[iw] : pad);
            }
        }
        uint32_t denom = g.ph * g.pw;
        if (!g.cip) denom = valid_taps(ih0, g.ph, g.dh, g.in_h) * valid_taps(iw0, g.pw, g.dw, g.in_w);
        yp[idx] = pool_finish(g.pool_type, g.lp_order, a.acc, denom);
    }
}

// ---------------------------------------------------------------- direct --
__global__ __launch_bounds__(kThreads) void pool_direct(const int16_t* __restrict__ x,
                                                        int16_t* __restrict__ y, PoolGeom g,
                                                        uint64_t total) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    const uint64_t ohw = (uint64_t)g.out_h * g.out_w;
    const int16_t pad = g.pool_type == CM_POOL_MAX ? (int16_t)-32768 : (int16_t)0;
    for (uint64_t o = (uint64_t)blockIdx.x * kThreads + threadIdx.x; o < total; o += stride) {
        const uint64_t plane = o / ohw;
        const uint32_t rem = (uint32_t)(o - plane * ohw);
        const uint32_t oh = rem / g.out_w, ow = rem - (rem / g.out_w) * g.out_w;
        const int16_t* xp = x + plane * (uint64_t)g.in_h * g.in_w;
        const int64_t ih0 = (int64_t)oh * g.sh - g.pt;
        const int64_t iw0 = (int64_t)ow * g.sw - g.pl;
        PoolAcc a;
        a.init(g.pool_type);
        for (uint32_t khi = 0; khi < g.ph; ++khi) {
            const int64_t ih = ih0 + (int64_t)khi * g.dh;
            const bool ih_ok = ih >= 0 && ih < (int64_t)g.in_h;
            for (uint32_t kwi = 0; kwi < g.pw; ++kwi) {
                const int64_t iw = iw0 + (int64_t)kwi * g.dw;
                const bool ok = ih_ok && iw >= 0 && iw < (int64_t)g.in_w;
                a.add(g.pool_type, g.lp_order, ok ? xp[(uint64_t)ih * g.in_w + iw] : pad);
            }
        }
        uint32_t denom = g.ph * g.pw;
        if (!g.cip) denom = valid_taps(ih0, g.ph, g.dh, g.in_h) * valid_taps(iw0, g.pw, g.dw, g.in_w);
        y[o] = pool_finish(g.pool_type, g.lp_order, a.acc, denom);
    }
}

// Input rows needed by `bh` consecutive output rows.
uint64_t rows_needed(const PoolGeom& g, uint32_t bh) {
    return (uint64_t)(bh - 1) * g.sh + (uint64_t)(g.ph - 1) * g.dh + 1;
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
    PoolGeom g{in_h, in_w, out_h, out_w, ph, pw, sh, sw, pad_top, pad_left, dh, dw,
               pool_type, lp_order, cip};
    if (ph == 0 || pw == 0 || in_h == 0 || in_w == 0) {
        // empty window or empty input: every output is the finaliser of the initial accumulator
        const uint64_t total = planes * out_h * out_w;
        hipLaunchKernelGGL(pool_direct, dim3((uint32_t)cm_grid_blocks(total, kThreads)),
                           dim3(kThreads), 0, s, x, y, g, total);
        return cm_check_launch("pool_direct");
    }
    const bool global = out_h == 1 && out_w == 1 && ph == in_h && pw == in_w && pad_top == 0 &&
                        pad_left == 0 && dh == 1 && dw == 1;
    if (global) {
        const uint64_t hw = (uint64_t)in_h * in_w;
        if (hw > 0xFFFFFFFFull) return cm_set_error(CM_ERR_RANGE, "pool: plane too large");
        const uint32_t vec_ok = (hw % 8 == 0) && (((uintptr_t)x & 15u) == 0);
        const uint64_t blocks = (planes + 3) / 4;
        if (blocks > 0x7FFFFFFFull) return cm_set_error(CM_ERR_RANGE, "pool: too many planes");
        hipLaunchKernelGGL(pool_global, dim3((uint32_t)blocks), dim3(kThreads), 0, s, x, y,
                           planes, (uint32_t)hw, pool_type, lp_order, (uint32_t)hw, vec_ok);
        return cm_check_launch("pool_global");
    }
    // band height: as many output rows as fit the LDS budget (+16 B alignment slack)
    uint32_t band_h = 0;
    const uint64_t row_bytes = (uint64_t)in_w * 2;
    if (rows_needed(g, 1) * row_bytes + 16 <= kLdsBytes) {
        uint32_t lo = 1, hi = out_h;
        while (lo < hi) {
            const uint32_t mid = lo + (hi - lo + 1) / 2;
            if (rows_needed(g, mid) * row_bytes + 16 <= kLdsBytes) lo = mid; else hi = mid - 1;
        }
        band_h = lo;
    }
    if (band_h > 0) {
        const uint32_t n_bands = (out_h + band_h - 1) / band_h;
        const uint64_t blocks = planes * n_bands;
        if (blocks <= 0x7FFFFFFFull) {
            uint64_t need = rows_needed(g, band_h);
            if (need > in_h) need = in_h;
            const uint32_t lds = (uint32_t)(need * row_bytes + 16);
            hipLaunchKernelGGL(pool_band, dim3((uint32_t)blocks), dim3(kThreads), lds, s, x, y,
                               g, band_h, n_bands);
            return cm_check_launch("pool_band");
        }
    }
    const uint64_t total = planes * out_h * out_w;
    hipLaunchKernelGGL(pool_direct, dim3((uint32_t)cm_grid_blocks(total, kThreads)),
                       dim3(kThreads), 0, s, x, y, g, total);
    return cm_check_launch("pool_direct");
}

int cm_finalize_sweep_launch(uint32_t mode, uint32_t lo, uint32_t count, uint32_t d,
                             unsigned long long* checksum, hipStream_t s) {
    hipLaunchKernelGGL(pool_finalize_sweep, dim3((uint32_t)cm_grid_blocks(count, kThreads, 4096)),
                       dim3(kThreads), 0, s, mode, lo, count, d, checksum);
    return cm_check_launch("pool_finalize_sweep");
}
