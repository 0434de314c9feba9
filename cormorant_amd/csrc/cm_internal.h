// cm_internal.h -- shared declarations of the gfx950 kernel library (not public).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cormorant_amd.h"   // include/: error codes, pool types

// VectorOP opcodes (kernels/vectorop/include/VectorOP.h:50-57); any other value copies a.
enum {
    CM_OP_ADD = 0,
    CM_OP_SUB = 1,
    CM_OP_MUL = 2,
    CM_OP_DIV = 3,
    CM_OP_RELU = 4,
    CM_OP_RELU6 = 5,
    CM_OP_COPY = 6,
};


int cm_set_error(int code, const char* fmt, ...);

// Where a MatMul / Conv launch runs and what scratch memory it may use.
//   ws / ws_bytes: the caller's workspace for split-K partial sums (null / 0 =
//     none: the call runs unsplit).  The library never allocates one.
//   need: dry run -- nothing is launched; *need is raised to the workspace
//     bytes the call would use with an unlimited workspace.
struct LaunchCtx {
    hipStream_t s;
    void* ws;
    size_t ws_bytes;
    size_t* need;
};

// Epilogue of a MatMul / Conv launch, flattened for kernel arguments:
// add_mode / act as in cm_epilogue_t (0 = none).
struct EpiArgs {
    const int16_t* add;
    uint32_t add_mode, act;
};
inline EpiArgs cm_epi_args(const cm_epilogue_t* e) {
    return e ? EpiArgs{e->add, e->add_mode, e->act} : EpiArgs{nullptr, 0u, 0u};
}
int cm_check_launch(const char* what);
bool cm_conv_gap_fits(uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch);
int cm_conv_gap_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                       uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch, uint32_t act,
                       hipStream_t s);
uint32_t cm_cu_count();   // compute units of the current device (cached per device)

// Division of any n < 2^31 by a fixed d >= 1 as a multiply and shift
// (Granlund-Montgomery, the round-up variant): l = ceil(log2 d), p = 31 + l,
// m = ceil(2^p / d) < 2^33; then n / d = (n * m) >> p exactly, since the
// error term n*(m*d - 2^p) / (d*2^p) stays below 2^-l <= 1/d.
struct FastDiv {
    uint32_t m_lo, m_hi, p;
};

inline FastDiv make_fastdiv(uint32_t d) {
    if (d == 0) d = 1;
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) ++l;
    const uint32_t p = 31 + l;
    const unsigned __int128 m = (((unsigned __int128)1 << p) + d - 1) / d;
    return FastDiv{(uint32_t)m, (uint32_t)(m >> 32), p};
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    // m_hi is 0 or 1: n * m_hi selects without a branch on the divisor
    const uint64_t t = (uint64_t)n * f.m_lo + ((uint64_t)(n * f.m_hi) << 32);
    return (uint32_t)(t >> f.p);
}

// Raw buffer resource word 3 for gfx950 (32-bit data, no swizzle): loads past
// num_records return 0 and stores past it are dropped.  kOob is an offset past
// every resource used here (all are smaller than 2^31 bytes).
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const int16_t* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<int16_t*>(base), (short)0, (int)bytes,
                                             kBufferWord3);
}

// Reads one dword of every 64-byte line that a struct kernel argument spans
// (offsets 0, 64, ... and its last dword) into one empty asm at a kernel's
// entry, so that all of the kernel's argument lines are requested at once.
// Read where first used, behind the branches that use them, each cold line
// costs a memory round trip of its own (one asm per line, or a chain of XORs,
// made the compiler wait between batches).  Struct parameters only: they are
// read in place in the argument segment (arithmetic across two parameters, or
// a scalar parameter's address, makes the compiler copy them to scratch).
template <typename A>
__device__ __forceinline__ void touch_lines(const A& a) {
    constexpr uint32_t n = sizeof(A) / 4;
    static_assert(sizeof(A) <= 7 * 64 + 4, "at most 8 argument lines");
    const uint32_t* d = reinterpret_cast<const uint32_t*>(&a);
    auto at = [&](uint32_t i) { return d[i * 16u < n ? i * 16u : n - 1u]; };
    asm volatile("" ::"s"(at(0)), "s"(at(1)), "s"(at(2)), "s"(at(3)), "s"(at(4)), "s"(at(5)),
                 "s"(at(6)), "s"(d[n - 1u]));
}
template <typename A, typename B>
__device__ __forceinline__ void touch_lines(const A& a, const B& b) {
    constexpr uint32_t na = sizeof(A) / 4, nb = sizeof(B) / 4;
    static_assert(sizeof(A) <= 196 && sizeof(B) <= 196, "at most 4 lines per argument");
    const uint32_t* da = reinterpret_cast<const uint32_t*>(&a);
    const uint32_t* db = reinterpret_cast<const uint32_t*>(&b);
    auto at = [](const uint32_t* d, uint32_t n, uint32_t i) { return d[i * 16u < n ? i * 16u : n - 1u]; };
    asm volatile("" ::"s"(at(da, na, 0)), "s"(at(da, na, 1)), "s"(at(da, na, 2)), "s"(da[na - 1u]),
                 "s"(at(db, nb, 0)), "s"(at(db, nb, 1)), "s"(at(db, nb, 2)), "s"(db[nb - 1u]));
}

inline uint64_t cm_grid_blocks(uint64_t work, uint32_t threads, uint64_t cap = 1u << 20) {
    uint64_t b = (work + threads - 1) / threads;
    if (b == 0) b = 1;
    return b > cap ? cap : b;
}

int cm_vectorop_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size,
                       uint32_t op, uint32_t outer, uint32_t a_inc, uint32_t b_inc,
                       hipStream_t s);
int cm_div_sweep_launch(uint32_t b_lo, uint32_t b_count, unsigned long long* out,
                        hipStream_t s);
int cm_pool_launch(const int16_t* x, int16_t* y, uint32_t batch, uint32_t ch, uint32_t in_h,
                   uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t ph, uint32_t pw,
                   uint32_t sh, uint32_t sw, uint32_t pad_top, uint32_t pad_left, uint32_t dh,
                   uint32_t dw, uint32_t pool_type, uint32_t lp_order, uint32_t cip,
                   hipStream_t s);
int cm_finalize_sweep_launch(uint32_t mode, uint32_t lo, uint32_t count, uint32_t d,
                             unsigned long long* checksum, hipStream_t s);
int cm_matmul_launch(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                     uint32_t m, uint32_t batch, uint32_t a_bs, uint32_t b_bs, uint32_t c_bs,
                     const cm_epilogue_t* epi, const LaunchCtx& lc);
// Convolution weights packed once for the patch-GEMM path (conv.hip,
// conv_pgemm.hip): the packed bytes for a shape (0 when cm_conv would not run
// it on that path), the pack, and a call that runs with packed weights.
size_t cm_conv_packed_bytes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                            uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                            uint32_t kw, uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
                            uint32_t pad_top, uint32_t pad_left, uint32_t is_dw);
size_t cm_conv_pgemm_packed_bytes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                                  uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                                  uint32_t kw, uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw,
                                  uint32_t pad_top, uint32_t pad_left);
int cm_conv_pgemm_pack(const int16_t* w, uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                       uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                       uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                       uint32_t pad_left, void* dst, size_t bytes, hipStream_t s);
int cm_conv_pgemm_run_packed(const int16_t* x, const void* packed, const int16_t* bias, int16_t* y,
                             uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                             uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                             uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                             uint32_t pad_left, const cm_epilogue_t* epi, hipStream_t s);
// A patch-GEMM convolution and a 1x1 convolution of its output in one launch
// (conv_pgemm.hip): packed-weight bytes (0 when the shapes do not take the
// path), the pack of both weight sets, and the run with them.
size_t cm_conv_pair_pgemm_bytes(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                                 uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                                 uint32_t kw, uint32_t stride, uint32_t dilation, uint32_t pad_top,
                                 uint32_t pad_left, uint32_t out_ch);
int cm_conv_pair_pgemm_pack(const int16_t* w1, const int16_t* w2, uint32_t batch, uint32_t in_ch, uint32_t in_h,
                      uint32_t in_w, uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                      uint32_t kw, uint32_t stride, uint32_t dilation, uint32_t pad_top, uint32_t pad_left,
                      uint32_t out_ch, void* dst, size_t bytes, hipStream_t s);
int cm_conv_pair_pgemm_run(const int16_t* x, const void* packed, const int16_t* bias1, const int16_t* bias2,
                            int16_t* y, uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                            uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                            uint32_t stride, uint32_t dilation, uint32_t pad_top, uint32_t pad_left,
                            uint32_t out_ch, uint32_t act1, const cm_epilogue_t* epi2, hipStream_t s);
// 3x3 convolution through an LDS-staged input patch (conv_patch.hip); returns
// 1, launching nothing, for shapes it does not take.
int cm_conv_patch_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                         uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                         uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                         uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                         uint32_t pad_left, const cm_epilogue_t* epi, const LaunchCtx& lc);
int cm_conv_launch(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                   uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                   uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                   uint32_t sh, uint32_t sw, uint32_t dh, uint32_t dw, uint32_t pad_top,
                   uint32_t pad_left, uint32_t has_bias, uint32_t is_dw, const cm_epilogue_t* epi,
                   const LaunchCtx& lc);
