// q88.h -- exact ap_fixed<16,8> / ap_fixed<32,16> arithmetic for gfx950 kernels.
//
// Data:        int16 raw r, value r/256 (kernels/*/CMakeLists.txt Data_t default).
// Accumulator: ap_fixed<32,16> raw bits carried in uint32 so that every "+="
//              wraps modulo 2^32 (AP_WRAP), value raw/65536.
// Output rule: saturate_cast<ap_fixed<16,8>> = AP_TRN floor (arithmetic >> 8
//              of the accumulator raw) then AP_SAT clamp to [-32768, 32767]
//              (kernels/vectorop/include/VectorOP.h:30-39).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q88 {

// IEEE binary32 round-to-nearest-even primitives.  The library is compiled
// with -ffp-contract=off, so a product is never fused into an FMA; division
// and square root lower to LLVM's correctly rounded fdiv / llvm.sqrt.f32
// expansions (no approximate-math flags).  The parity tests sweep every
// accumulator value of both finalisers against the host's float32 results.
__device__ __forceinline__ float mul_rn(float x, float y) { return x * y; }
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ float div_rn(float x, float y) { return x / y; }

// PoolingKernel.cpp:137: inv_denom = denom > 0 ? 1.0f / (float)denom : 0.0f
__device__ __forceinline__ float inv_denom(uint32_t d) {
    return d > 0u ? div_rn(1.0f, (float)d) : 0.0f;
}

__device__ __forceinline__ int32_t sat16(int32_t v) {
    return __builtin_elementwise_min(__builtin_elementwise_max(v, -32768), 32767);
}

// saturate_cast<Data_t>(AccData_t acc)
__device__ __forceinline__ int16_t acc_to_data(uint32_t acc) {
    return (int16_t)sat16(((int32_t)acc) >> 8);
}

// Data_t -> AccData_t (raw << 8)
__device__ __forceinline__ uint32_t data_to_acc(int32_t x) { return (uint32_t)x << 8; }

// VectorOP.cpp:8-14: sat16(a + b), sat16(a - b)
__device__ __forceinline__ int32_t add(int32_t a, int32_t b) { return sat16(a + b); }
__device__ __forceinline__ int32_t sub(int32_t a, int32_t b) { return sat16(a - b); }

// VectorOP.cpp:17-19: full-precision product, AP_TRN floor of 8 bits, AP_SAT.
__device__ __forceinline__ int32_t mul(int32_t a, int32_t b) { return sat16((a * b) >> 8); }

// VectorOP.cpp:22-25: b == 0 -> 0, else sat16(trunc((a * 256) / b)).
// Branch-free in float, on magnitudes: X = 256 |a| and B = |b| are exact
// floats (X < 2^23; B = 1 stands in for b == 0, masked at the end).  The
// estimate q0 = floor(X * rcp(B)) (v_rcp_f32, within one ulp) is within two of
// floor(X / B); the remainder r = X - q0 B comes from one FMA and is exact (an
// integer, |r| < 3B), and floor(r * rcp(B) + 2^-18) is exactly the number of
// steps q0 is off: r / B lies at least 1/B >= 2^-15 below any integer it does
// not reach, far more than the product's rounding error (< 2^-20) plus the
// 2^-18 nudge, and the nudge lifts a product that rounds just under an integer
// r / B equals.  The sign of a ^ b then goes onto the magnitude.  Verified
// exhaustively over all 2^32 (a, b) pairs against exact division, on the GPU
// and on the CPU with the reciprocal moved up to three ulps either way.
// div_q is the unsaturated quotient (|q| <= 2^23, 0 for b == 0).
__device__ __forceinline__ int32_t div_q(int32_t a, int32_t b) {
    const float B = __builtin_fmaxf(__builtin_fabsf((float)b), 1.0f);
    const float X = __builtin_fabsf((float)a) * 256.0f;
    const float rb = __builtin_amdgcn_rcpf(B);
    const float q0 = __builtin_floorf(X * rb);
    const float r = __builtin_fmaf(-q0, B, X);
    const float q = q0 + __builtin_floorf(__builtin_fmaf(r, rb, 0x1p-18f));
    const uint32_t qs = __builtin_bit_cast(uint32_t, q) | ((uint32_t)(a ^ b) & 0x80000000u);
    return (int32_t)__builtin_bit_cast(float, qs) & -(int32_t)(b != 0);
}
__device__ __forceinline__ int32_t div(int32_t a, int32_t b) { return sat16(div_q(a, b)); }
// Two quotients saturated and packed by one v_cvt_pk_i16_i32: (a0 / b0) in the
// low half, (a1 / b1) in the high half.
__device__ __forceinline__ uint32_t div2(int32_t a0, int32_t b0, int32_t a1, int32_t b1) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(div_q(a0, b0), div_q(a1, b1)));
}

// VectorOP.cpp:27-35
__device__ __forceinline__ int32_t relu(int32_t a) { return a < 0 ? 0 : a; }
__device__ __forceinline__ int32_t relu6(int32_t a) {
    return a < 0 ? 0 : (a > 1536 ? 1536 : a);
}

// Fused epilogue activation (cm_epilogue_t act): 1 = RELU, 2 = RELU6, else none.
__device__ __forceinline__ int32_t epi_act(int32_t y, uint32_t act) {
    return act == 1u ? relu(y) : (act == 2u ? relu6(y) : y);
}

// The same activation as clamp bounds for a saturated value y: RELU = [0, 32767],
// RELU6 = [0, 1536], none = the full int16 range.  Computed once, it turns the
// per-value choice into one min / max pair with no branch.
__device__ __forceinline__ int32_t act_lo(uint32_t act) { return act == 1u || act == 2u ? 0 : -32768; }
__device__ __forceinline__ int32_t act_hi(uint32_t act) { return act == 2u ? 1536 : 32767; }
__device__ __forceinline__ int32_t clamp(int32_t y, int32_t lo, int32_t hi) {
    return __builtin_elementwise_min(__builtin_elementwise_max(y, lo), hi);
}

// (float)AccData_t: nearest-even rounding of raw, then exact scale by 2^-16.
__device__ __forceinline__ float acc_to_float(uint32_t acc) {
    return mul_rn((float)(int32_t)acc, 1.0f / 65536.0f);   // v_cvt_f32_i32 rounds to nearest even
}

// saturate_cast<Data_t>(AccData_t(f)) for |f| < 32768: AccData_t floors f to a
// multiple of 2^-16 and the output keeps floor(f * 256), saturated (the scale is
// exact).  Both pool finalisers stay in that range (see below).
__device__ __forceinline__ int16_t floor_to_data(float f256) {   // f256 = f * 256
    const float s = __builtin_amdgcn_fmed3f(__builtin_floorf(f256), -8388608.0f, 8388607.0f);
    return (int16_t)sat16((int32_t)s);
}
__device__ __forceinline__ int16_t float_to_data(float f) { return floor_to_data(mul_rn(f, 256.0f)); }

// PoolingKernel.cpp:137, 259, 265: AccData_t((float)acc * (1.0f / denom)).
// |acc * 2^-16| <= 32768, times 1/d <= 1/2 for d >= 2; for d = 1 the sum is one
// value << 8, so |f| <= 128; d = 0 gives 0: the result is always in range.
// The reference's floor(fl32(fl32(raw) * 2^-16 * inv) * 256) is computed as
// floor(fl32(fl32(raw) * inv8)) with inv8 = inv * 2^-8: power-of-two scalings
// commute with rounding away from the subnormal range (|fl32(raw) * inv| is 0
// or at least 2^-32 here), so both give the same float for every accumulator.
__device__ __forceinline__ int16_t avg_finalize8(uint32_t acc, float inv8) {
    return floor_to_data(mul_rn((float)(int32_t)acc, inv8));
}
__device__ __forceinline__ int16_t avg_finalize(uint32_t acc, float inv_denom) {
    return avg_finalize8(acc, mul_rn(inv_denom, 1.0f / 256.0f));
}

// Correctly rounded square root of x = 0 or a normal x (the LP accumulator's
// raw value as a float: 0 or at least 1): the hardware estimate, within one ulp, moved to
// the nearest float by the signs of the residuals x - n * s of its neighbours n
// (the same correction LLVM's IEEE square root applies, without its rescaling
// of subnormal inputs).  Negative x gives NaN.
__device__ __forceinline__ float sqrt_acc(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float dn = __builtin_bit_cast(float, __builtin_bit_cast(int32_t, s) - 1);
    const float up = __builtin_bit_cast(float, __builtin_bit_cast(int32_t, s) + 1);
    float r = __builtin_fmaf(-dn, s, x) <= 0.0f ? dn : s;
    r = __builtin_fmaf(-up, s, x) > 0.0f ? up : r;
    return r;
}

// PoolingKernel.cpp:263, 265: AccData_t(sqrtf((float)acc)), kept as floor(root *
// 256) saturated.  With a = fl32(raw), sqrtf(a * 2^-16) * 256 = RN(sqrt(a)) exactly
// (power-of-two scalings commute with the rounding), and a non-negative root is
// floored by truncation; it reaches at most 46341, so only the top clamp applies.
// A negative (wrapped) sum's root is NaN, which the reference's conversion takes
// to 0 (selected, not branched: the pool kernels keep every load in flight past it).
__device__ __forceinline__ int16_t lp2_finalize(uint32_t acc) {
    const int32_t r = (int32_t)sqrt_acc((float)(int32_t)acc);   // NaN only when acc < 0
    return (int32_t)acc < 0 ? (int16_t)0 : (int16_t)__builtin_elementwise_min(r, 32767);
}

}  // namespace q88
