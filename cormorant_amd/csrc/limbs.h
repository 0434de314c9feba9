// limbs.h -- int8 limb helpers shared by the register-only MFMA convolutions.
//
// A Q8.8 value v (int16) splits into a signed high byte and an offset low
// byte, both int8: vh = v >> 8, vl = (v & 255) - 128, v = 256*vh + vl + 128.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace limbs {

// High / low limb bytes of four int16 values held in two words w0 = (v0 | v1 << 16),
// w1 = (v2 | v3 << 16); byte i of the result belongs to value i (k order kept).
__device__ __forceinline__ uint32_t hi4(uint32_t w0, uint32_t w1) {
    return __builtin_amdgcn_perm(w1, w0, 0x07050301u);
}
__device__ __forceinline__ uint32_t lo4(uint32_t w0, uint32_t w1) {
    return __builtin_amdgcn_perm(w1, w0, 0x06040200u) ^ 0x80808080u;
}
// Sum of the four signed bytes of w added to acc.
__device__ __forceinline__ int32_t bsum(uint32_t w, int32_t acc) {
    return __builtin_amdgcn_sdot4((int)w, 0x01010101, acc, false);
}
// Two zero-extended int16 values -> one word (lo | hi << 16).
__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

}  // namespace limbs
