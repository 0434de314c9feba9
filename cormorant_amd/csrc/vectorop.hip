// vectorop.hip -- VectorOPKernel for gfx950 (kernels/vectorop/kernel/VectorOP.cpp:140-188).
//
//   c[o*(a_inc+b_inc) + i] = op(a[o*a_inc + i], b[o*b_inc + i]),  o < outer, i < size
//
// HBM-streaming design: every thread moves whole 16-byte vectors (8 Q8.8
// values) with UNROLL independent loads in flight; unary ops never touch b.
// Three launch shapes:
//   * flat      (outer == 1 or a contiguous broadcast that is really flat):
//               1-D grid over 16-byte vectors, scalar tail handled by one block;
//   * rows      (outer > 1, rows 16-byte aligned, no overlapping outputs):
//               grid over (row, vector-in-row) with 16-byte accesses;
//   * ordered   (anything else: unaligned rows or outputs of different outer
//               steps overlapping): one thread per output element, which picks
//               the LAST outer step that writes it -- the state the reference's
//               sequential outer loop leaves behind.
#include "cm_internal.h"
#include "q88.h"

namespace {

typedef short v8s __attribute__((ext_vector_type(8)));

template <int OP>
__device__ __forceinline__ int32_t apply(int32_t a, int32_t b) {
    if constexpr (OP == CM_OP_ADD) return q88::add(a, b);
    else if constexpr (OP == CM_OP_SUB) return q88::sub(a, b);
    else if constexpr (OP == CM_OP_MUL) return q88::mul(a, b);
    else if constexpr (OP == CM_OP_DIV) return q88::div(a, b);
    else if constexpr (OP == CM_OP_RELU) return q88::relu(a);
    else if constexpr (OP == CM_OP_RELU6) return q88::relu6(a);
    else return a;   // any other opcode copies a (VectorOP.cpp:112)
}

template <int OP>
__device__ __forceinline__ v8s apply8(v8s a, v8s b) {
    if constexpr (OP == CM_OP_DIV) {
        // unsaturated quotients, saturated and packed two at a time
        typedef unsigned int v4u8 __attribute__((ext_vector_type(4)));
        v4u8 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const short a0 = a[2 * j], a1 = a[2 * j + 1], b0 = b[2 * j], b1 = b[2 * j + 1];
            r[j] = q88::div2(a0, b0, a1, b1);
        }
        return __builtin_bit_cast(v8s, r);
    } else {
        v8s r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (short)apply<OP>(a[j], b[j]);
        return r;
    }
}

constexpr bool is_binary(int op) { return op < CM_OP_RELU; }

constexpr int kThreads = 256;
// 16-byte vectors per thread (all loads issued before any op): 2 measured best
// on the 64 Mi sweep -- DIV, whose per-element work keeps a wave longer between
// its loads and its stores, 69 us against 73-75 us at 4; the other ops equal
constexpr int kUnroll = 2;

// Flat stream over nvec 16-byte vectors + a scalar tail of `tail` elements.
template <int OP>
__global__ __launch_bounds__(kThreads) void vecop_flat(const v8s* __restrict__ a,
                                                       const v8s* __restrict__ b,
                                                       v8s* __restrict__ c, uint64_t nvec,
                                                       uint32_t tail) {
    const uint64_t base = (uint64_t)blockIdx.x * (kThreads * kUnroll) + threadIdx.x;
    if (base < nvec) {
        v8s va[kUnroll], vb[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t idx = base + (uint64_t)u * kThreads;
            if (idx < nvec) {
                va[u] = __builtin_nontemporal_load(a + idx);
                if constexpr (is_binary(OP)) vb[u] = __builtin_nontemporal_load(b + idx);
                else vb[u] = v8s{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t idx = base + (uint64_t)u * kThreads;
            if (idx < nvec) __builtin_nontemporal_store(apply8<OP>(va[u], vb[u]), c + idx);
        }
    }
    if (tail != 0 && blockIdx.x == gridDim.x - 1 && threadIdx.x < tail) {
        const int16_t* as = reinterpret_cast<const int16_t*>(a + nvec);
        const int16_t* bs = reinterpret_cast<const int16_t*>(b + nvec);
        int16_t* cs = reinterpret_cast<int16_t*>(c + nvec);
        const int32_t bv = is_binary(OP) ? (int32_t)bs[threadIdx.x] : 0;
        cs[threadIdx.x] = (int16_t)apply<OP>(as[threadIdx.x], bv);
    }
}

// Broadcast rows, all row starts 16-byte aligned and size % 8 == 0.
template <int OP>
__global__ __launch_bounds__(kThreads) void vecop_rows(const v8s* __restrict__ a,
                                                       const v8s* __restrict__ b,
                                                       v8s* __restrict__ c, uint32_t vec_per_row,
                                                       uint32_t outer, uint64_t a_inc_v,
                                                       uint64_t b_inc_v, uint64_t c_inc_v) {
    const uint64_t total = (uint64_t)vec_per_row * outer;
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    for (uint64_t t = (uint64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += stride) {
        const uint64_t o = t / vec_per_row;
        const uint64_t v = t - o * vec_per_row;
        const v8s va = a[o * a_inc_v + v];
        const v8s vb = is_binary(OP) ? b[o * b_inc_v + v] : v8s{0, 0, 0, 0, 0, 0, 0, 0};
        c[o * c_inc_v + v] = apply8<OP>(va, vb);
    }
}

// Output-centric general form.  Output position p is written by outer steps
// o with o*c_inc <= p < o*c_inc + size; the sequential reference leaves the
// value of the largest such o.  Gap positions (no writer) are untouched.
template <int OP>
__global__ __launch_bounds__(kThreads) void vecop_ordered(const int16_t* __restrict__ a,
                                                          const int16_t* __restrict__ b,
                                                          int16_t* __restrict__ c, uint32_t size,
                                                          uint32_t outer, uint64_t a_inc,
                                                          uint64_t b_inc, uint64_t c_inc,
                                                          uint64_t span) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    for (uint64_t p = (uint64_t)blockIdx.x * kThreads + threadIdx.x; p < span; p += stride) {
        uint64_t o = outer - 1;
        if (c_inc != 0) {
            const uint64_t q = p / c_inc;
            o = q < o ? q : o;
        }
        const uint64_t i = p - o * c_inc;
        if (i >= size) continue;
        const int32_t av = a[o * a_inc + i];
        const int32_t bv = is_binary(OP) ? (int32_t)b[o * b_inc + i] : 0;
        c[p] = (int16_t)apply<OP>(av, bv);
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int OP>
int launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size, uint32_t outer,
           uint32_t a_inc, uint32_t b_inc, hipStream_t s) {
    const uint64_t c_inc = (uint64_t)a_inc + b_inc;
    const bool bin = is_binary(OP);
    // outer == 1, or a unary op whose rows tile a and c back to back: one flat stream.
    const bool flat = outer == 1 || (!bin && a_inc == size && b_inc == 0);
    const uint64_t n = flat ? (uint64_t)size * outer : 0;
    if (flat && aligned16(a) && aligned16(c) && (!bin || aligned16(b))) {
        const uint64_t nvec = n / 8;
        const uint32_t tail = (uint32_t)(n % 8);
        uint64_t blocks = (nvec + kThreads * kUnroll - 1) / (kThreads * kUnroll);
        if (blocks == 0) blocks = 1;
        hipLaunchKernelGGL(vecop_flat<OP>, dim3((uint32_t)blocks), dim3(kThreads), 0, s,
                           reinterpret_cast<const v8s*>(a), reinterpret_cast<const v8s*>(b),
                           reinterpret_cast<v8s*>(c), nvec, tail);
        return cm_check_launch("vectorop_flat");
    }
    const bool rows_ok = outer > 1 && (size % 8) == 0 && (a_inc % 8) == 0 &&
                         (!bin || (b_inc % 8) == 0) && (c_inc % 8) == 0 && c_inc >= size &&
                         aligned16(a) && aligned16(c) && (!bin || aligned16(b));
    if (rows_ok) {
        const uint64_t total = (uint64_t)(size / 8) * outer;
        const uint64_t blocks = cm_grid_blocks(total, kThreads);
        hipLaunchKernelGGL(vecop_rows<OP>, dim3((uint32_t)blocks), dim3(kThreads), 0, s,
                           reinterpret_cast<const v8s*>(a), reinterpret_cast<const v8s*>(b),
                           reinterpret_cast<v8s*>(c), size / 8, outer, (uint64_t)a_inc / 8,
                           (uint64_t)b_inc / 8, c_inc / 8);
        return cm_check_launch("vectorop_rows");
    }
    const uint64_t span = (uint64_t)(outer - 1) * c_inc + size;
    const uint64_t blocks = cm_grid_blocks(span, kThreads);
    hipLaunchKernelGGL(vecop_ordered<OP>, dim3((uint32_t)blocks), dim3(kThreads), 0, s, a, b, c,
                       size, outer, (uint64_t)a_inc, (uint64_t)b_inc, c_inc, span);
    return cm_check_launch("vectorop_ordered");
}

}  // namespace

int cm_vectorop_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size,
                       uint32_t op, uint32_t outer, uint32_t a_inc, uint32_t b_inc,
                       hipStream_t s) {
    switch (op) {
    case CM_OP_ADD: return launch<CM_OP_ADD>(a, b, c, size, outer, a_inc, b_inc, s);
    case CM_OP_SUB: return launch<CM_OP_SUB>(a, b, c, size, outer, a_inc, b_inc, s);
    case CM_OP_MUL: return launch<CM_OP_MUL>(a, b, c, size, outer, a_inc, b_inc, s);
    case CM_OP_DIV: return launch<CM_OP_DIV>(a, b, c, size, outer, a_inc, b_inc, s);
    case CM_OP_RELU: return launch<CM_OP_RELU>(a, b, c, size, outer, a_inc, b_inc, s);
    case CM_OP_RELU6: return launch<CM_OP_RELU6>(a, b, c, size, outer, a_inc, b_inc, s);
    default: return launch<CM_OP_COPY>(a, b, c, size, outer, a_inc, b_inc, s);
    }
}

// Exhaustive check of the DIV estimate-and-correct path against integer
// division over every (a, b) int16 pair; counts mismatches into *mismatches.
// out[0] counts mismatches; out[1] keeps one mismatching case packed as
// (a << 48) | (b << 32) | (got << 16) | want (16-bit fields, 0 if none).
__global__ __launch_bounds__(kThreads) void vecop_div_sweep(uint32_t b_lo, uint32_t b_count,
                                                            unsigned long long* out) {
    const uint32_t b_idx = blockIdx.y + b_lo;
    if (b_idx >= b_lo + b_count || b_idx > 0xFFFFu) return;
    const int32_t bv = (int16_t)(uint16_t)b_idx;
    const int32_t av = (int16_t)(uint16_t)(blockIdx.x * kThreads + threadIdx.x);
    // Reference value from double-precision division.  Integer division is
    // not usable here: the compiler narrows a 32- or 64-bit signed division
    // whose operands fit 24 bits to a 24-bit sequence, and that sequence
    // returns -2^23 for (-2^23) / (-1).  In double, A / b (|A| <= 2^23,
    // |b| <= 2^15) lies at least 2^-15 away from any integer it is not equal
    // to, far above the 2^-30 rounding error, so trunc() is exact.
    int32_t want = 0;
    if (bv != 0) {
        const double q = __builtin_trunc((double)(av * 256) / (double)bv);
        want = (int32_t)(q > 32767.0 ? 32767.0 : (q < -32768.0 ? -32768.0 : q));
    }
    // the packed pair form the streaming kernel runs: (av, bv) in the low half,
    // and the scalar form beside it
    const uint32_t pair = q88::div2(av, bv, av, bv);
    const int32_t got_lo = (int16_t)(pair & 0xFFFFu), got_hi = (int32_t)pair >> 16;
    const int32_t got_s = q88::div(av, bv);
    const int32_t got = got_lo != want ? got_lo : (got_hi != want ? got_hi : got_s);
    const unsigned long long bad = __ballot(got != want);
    if ((threadIdx.x & 63) == 0 && bad != 0) atomicAdd(out, (unsigned long long)__popcll(bad));
    if (got != want) {
        const unsigned long long rec = ((unsigned long long)(uint16_t)av << 48) |
                                       ((unsigned long long)(uint16_t)bv << 32) |
                                       ((unsigned long long)(uint16_t)got << 16) | (uint16_t)want;
        atomicMax(out + 1, rec);
    }
}

int cm_div_sweep_launch(uint32_t b_lo, uint32_t b_count, unsigned long long* out,
                        hipStream_t s) {
    hipLaunchKernelGGL(vecop_div_sweep, dim3(65536 / kThreads, b_count), dim3(kThreads), 0, s,
                       b_lo, b_count, out);
    return cm_check_launch("vectorop_div_sweep");
}
