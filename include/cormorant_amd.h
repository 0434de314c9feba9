/*
 * cormorant_amd.h -- C ABI of the MI355X (gfx950) implementation of Cormorant's
 * four Q8.8 inference kernels: VectorOPKernel, MatmulKernel, ConvKernel and
 * PoolingKernel.
 *
 * Data: every tensor is int16 two's complement holding ap_fixed<16,8>
 * (value = raw / 256), NCHW for conv/pool, row-major for matmul.  Results are
 * bit-identical to the reference C-simulation kernels, including the 32-bit
 * wrapping accumulator and the truncate-then-saturate output rule.
 *
 * Conventions
 *   - Kernel entry points take DEVICE pointers and enqueue work on `stream`
 *     (NULL = the library stream set by cm_set_stream, default stream 0); they
 *     return as soon as the work is queued.  Results are visible after
 *     cm_sync() or cm_buf_sync_from_device().  One in-order stream gives the
 *     reference's strictly sequential node order.
 *   - Every function returning int returns 0 on success and a negative CM_ERR_*
 *     code otherwise; cm_last_error() describes the last failure of the
 *     calling thread.  Where the reference has undefined behaviour (shapes
 *     beyond its compile-time kMax* limits) this library computes the exact
 *     result instead, or returns CM_ERR_RANGE if a size exceeds its indexing.
 *   - The caller owns every buffer, and no entry point allocates device
 *     memory (cm_buf_alloc is the allocator, as inference_buf_alloc is in the
 *     reference).  A MatMul / Conv call whose output tiles are too few to
 *     fill the GPU can split its k range over extra blocks and add the
 *     partial sums in a second pass, and a large MatMul (at least 256 output
 *     tiles of 128 x 128, K <= 32768, K and M multiples of 8, 16-byte aligned
 *     operands) packs its B operand into MFMA-ready limb fragments once per
 *     call; the partials and the packed B go to a WORKSPACE the caller provides: per call (cm_matmul_ex / cm_conv_ex) or as the default
 *     for calls that take none (cm_set_workspace).  The size a call would use
 *     is returned by cm_matmul_workspace_size / cm_conv_workspace_size; a
 *     smaller workspace gives fewer splits, none gives none -- the result is
 *     the same bit for bit, only the speed differs.  The sizes assume a
 *     16-byte-aligned workspace (a cm_buf_t's device memory and torch's
 *     allocations are 256-byte aligned); at another address a MatMul uses it
 *     from its first 16-byte-aligned byte on, and a Conv runs a path that
 *     needs none -- again the same result, only slower.
 *     Calls that may run at
 *     the same time (different streams, a replayed HIP graph beside eager
 *     work) must not share a workspace; calls queued on one stream may.
 *
 * Reference interfaces replaced (paths relative to the reference root):
 *   kernels/vectorop/include/VectorOP.h:86-95        VectorOPKernel
 *   kernels/matmul/include/MatmulKernel.h:68-79      MatmulKernel
 *   kernels/conv/include/ConvKernel.h:79-101         ConvKernel
 *   kernels/pool/include/PoolingKernel.h:63-83       PoolingKernel
 *   inference-scheduler/src/codegen/_source.py:198-421  run_op / run_matmul /
 *       run_matmul_at / run_conv / run_pool (generated C helpers)
 *   inference-scheduler/bench_src/inference.h:12-38  inference_buf_* (DMA buffers)
 */
#ifndef CORMORANT_AMD_H
#define CORMORANT_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. */
#define CM_OK          0
#define CM_ERR_INVALID (-1)  /* null pointer or inconsistent arguments */
#define CM_ERR_HIP     (-2)  /* HIP runtime / launch failure */
#define CM_ERR_RANGE   (-3)  /* size beyond the library's indexing */
#define CM_ERR_NOMEM   (-4)  /* allocation failed */

/* VectorOP opcodes: kernels/vectorop/include/VectorOP.h:50-57.
 * Any other opcode copies a (kernels/vectorop/kernel/VectorOP.cpp:112). */
#define CM_VECTOROP_ADD   0u
#define CM_VECTOROP_SUB   1u
#define CM_VECTOROP_MUL   2u
#define CM_VECTOROP_DIV   3u
#define CM_VECTOROP_RELU  4u
#define CM_VECTOROP_RELU6 5u

/* Pool types: kernels/pool/include/Config.h.in:40-42.  Any other value is Lp. */
#define CM_POOL_MAX 0u
#define CM_POOL_AVG 1u
#define CM_POOL_LP  2u

/* ------------------------------------------------------------------ kernels */

/* VectorOPKernel (VectorOP.h:86-95):
 *   c[o*(a_inc+b_inc) + i] = op(a[o*a_inc + i], b[o*b_inc + i]),
 *   o < outer, i < size.  b may be NULL for op RELU/RELU6 (never read).
 * Overlapping outputs of different outer steps keep the last step's value. */
int cm_vectorop(const int16_t *a, const int16_t *b, int16_t *c, uint32_t size, uint32_t op,
                uint32_t outer, uint32_t a_inc, uint32_t b_inc, hipStream_t stream);

/* MatmulKernel (MatmulKernel.h:68-79): for bi < batch,
 *   C_bi[n][m] = sat16(wrap32(sum_k A_bi[n][k] * B_bi[k][m]) >> 8)
 * with A_bi = a + bi*a_stride, B_bi = b + bi*b_stride, C_bi = c + bi*c_stride
 * (element strides; 0 broadcasts).  No limit on k (the reference's kMaxK=2048
 * static buffer is not needed); k = 0 gives 0.  Batches run in order: where
 * the outputs of two batches overlap (c_stride < n*m) an element keeps the
 * value of the last batch that writes it, as in the reference's sequential
 * batch loop (MatmulKernel.cpp:108-111).  Uses the default workspace. */
int cm_matmul(const int16_t *a, const int16_t *b, int16_t *c, uint32_t n, uint32_t k,
              uint32_t m, uint32_t batch, uint32_t a_stride, uint32_t b_stride,
              uint32_t c_stride, hipStream_t stream);

/* run_matmul_at (_source.py:275-300): cm_matmul on a+a_off, b+b_off, c+c_off. */
int cm_matmul_at(const int16_t *a, uint32_t a_off, const int16_t *b, uint32_t b_off,
                 int16_t *c, uint32_t c_off, uint32_t n, uint32_t k, uint32_t m,
                 uint32_t batch, uint32_t a_stride, uint32_t b_stride, uint32_t c_stride,
                 hipStream_t stream);

/* ConvKernel (ConvKernel.h:79-101): NCHW, weights [out_ch][in_ch][kh][kw]
 * (depthwise: [out_ch][1][kh][kw], output channel m reads input channel m),
 * bias [out_ch] (NULL allowed when has_bias == 0), pad_bottom/right implicit.
 * Depthwise requires out_ch <= in_ch.  Uses the default workspace. */
int cm_conv(const int16_t *x, const int16_t *weight, const int16_t *bias, int16_t *y,
            uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
            uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
            uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
            uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, hipStream_t stream);

/* PoolingKernel (PoolingKernel.h:63-83): MAX / AVG / LP(lp_order 1, else 2),
 * Global variants by passing the whole plane as the window. */
int cm_pool(const int16_t *x, int16_t *y, uint32_t batch, uint32_t channels, uint32_t in_h,
            uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t pool_h, uint32_t pool_w,
            uint32_t stride_h, uint32_t stride_w, uint32_t pad_top, uint32_t pad_left,
            uint32_t dil_h, uint32_t dil_w, uint32_t pool_type, uint32_t lp_order,
            uint32_t count_include_pad, hipStream_t stream);

/* ---------------------------------------------------------- fused epilogues */

/* Element-wise epilogue applied by a MatMul / Conv call to each output value y
 * (the saturated Q8.8 result) before it is stored:
 *   add_mode CM_EPI_ADD_SAME:   y = sat16(y + add[i]), add laid out exactly like
 *                               the output (same strides; add == output is allowed);
 *   add_mode CM_EPI_ADD_COLUMN: y = sat16(y + add[j]) for output column j
 *                               (MatMul only: a bias row broadcast over rows and batches);
 *   then act CM_EPI_ACT_RELU:   y = max(y, 0);  CM_EPI_ACT_RELU6: y = clamp(y, 0, 1536).
 * The stored value equals what run_op(ADD) and then run_op(RELU / RELU6) would
 * leave when applied to the unfused output (VectorOP.cpp:8-35).  add must not
 * overlap the call's inputs or any other part of its output. */
#define CM_EPI_ADD_NONE   0u
#define CM_EPI_ADD_SAME   1u
#define CM_EPI_ADD_COLUMN 2u
#define CM_EPI_ACT_NONE   0u
#define CM_EPI_ACT_RELU   1u
#define CM_EPI_ACT_RELU6  2u

typedef struct cm_epilogue {
    const int16_t *add;   /* NULL when add_mode == CM_EPI_ADD_NONE */
    uint32_t add_mode;
    uint32_t act;
} cm_epilogue_t;

/* cm_matmul / cm_conv with an epilogue (epi may be NULL = none) and a
 * workspace of workspace_bytes bytes at device address `workspace` (NULL = no
 * split-K).  No reference counterpart: they let a caller such as the
 * scheduler's GPU backend fold the run_op Add / Relu / Clip(0,6) that follows
 * a run_matmul / run_conv into that call, saving a launch and a round trip of
 * the intermediate through memory, and keep split-K scratch in the caller's
 * own pool (the reference's one-allocation buffer plan, _source.py:494-505). */
int cm_matmul_ex(const int16_t *a, const int16_t *b, int16_t *c, uint32_t n, uint32_t k,
                 uint32_t m, uint32_t batch, uint32_t a_stride, uint32_t b_stride,
                 uint32_t c_stride, const cm_epilogue_t *epi, void *workspace,
                 size_t workspace_bytes, hipStream_t stream);
int cm_conv_ex(const int16_t *x, const int16_t *weight, const int16_t *bias, int16_t *y,
               uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
               uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
               uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
               uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise,
               const cm_epilogue_t *epi, void *workspace, size_t workspace_bytes,
               hipStream_t stream);

/* Workspace bytes the call with these arguments uses for its split-K partial
 * sums when given enough (0 = it never splits).  No reference counterpart; no
 * GPU work.  A workspace of the largest size over a sequence of calls serves
 * every call of the sequence on one stream. */
size_t cm_matmul_workspace_size(uint32_t n, uint32_t k, uint32_t m, uint32_t batch,
                                uint32_t a_stride, uint32_t b_stride, uint32_t c_stride);
size_t cm_conv_workspace_size(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                              uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                              uint32_t kw, uint32_t stride_h, uint32_t stride_w,
                              uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                              uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise);

/* Weights packed once, for callers that run one convolution's weights many
 * times (an inference session loading a model).  No reference counterpart:
 * cm_conv / cm_conv_ex repack the weights on every call, as ConvKernel reads
 * them on every call.  cm_conv_packed_size returns the bytes of the packed
 * weights for a shape that cm_conv runs on its patch-GEMM path (windows of two
 * or more taps, the same stride and dilation on both axes), and 0 for any
 * other shape; cm_conv_pack writes them (into caller-owned, 16-byte aligned
 * device memory); cm_conv_packed_ex then computes exactly what cm_conv_ex
 * computes with the weights that were packed, without repacking.  The packed
 * bytes depend on in_ch, out_ch, kh and kw only; any other argument may change
 * between cm_conv_pack and cm_conv_packed_ex as long as the shape still takes
 * the path (cm_conv_packed_size > 0). */
size_t cm_conv_packed_size(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                           uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                           uint32_t kw, uint32_t stride_h, uint32_t stride_w,
                           uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                           uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise);
int cm_conv_pack(const int16_t *weight, uint32_t batch, uint32_t in_ch, uint32_t in_h,
                 uint32_t in_w, uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                 uint32_t kw, uint32_t stride_h, uint32_t stride_w, uint32_t dilation_h,
                 uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left, uint32_t has_bias,
                 uint32_t is_depthwise, void *packed, size_t packed_bytes, hipStream_t stream);
int cm_conv_packed_ex(const int16_t *x, const void *packed, const int16_t *bias, int16_t *y,
                      uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                      uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                      uint32_t stride_h, uint32_t stride_w, uint32_t dilation_h,
                      uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left,
                      uint32_t has_bias, uint32_t is_depthwise, const cm_epilogue_t *epi,
                      hipStream_t stream);

/* A convolution and a 1x1 convolution of its output in one launch.  No
 * counterpart in the reference, where they are two run_conv calls (with a
 * run_op for the activation between them and one for a residual Add after):
 * the scheduler session uses it for Conv -> Relu/Clip(0,6) -> Conv 1x1 chains
 * whose middle tensor nothing else reads.  The first convolution: x
 * [batch][in_ch][in_h][in_w], weights w1 [mid_ch][in_ch][kh][kw], the same
 * stride and dilation on both axes, padding pad_top / pad_left, optional
 * bias1, then act1 (0 none, 1 Relu, 2 Clip(0,6)); the second: weights w2
 * [out_ch][mid_ch], optional bias2, then epi2 (a same-shaped Add and / or an
 * activation); y [batch][out_ch][out_h][out_w].  The middle tensor stays in
 * LDS.  cm_conv_pair_packed_size returns the packed-weight bytes (0 when the
 * shapes do not take the path: mid_ch at most 128 and out_ch at most 256,
 * and the first convolution's input rows must fit the kernel's LDS patch);
 * cm_conv_pair_pack writes both weight sets (16-byte aligned device memory);
 * cm_conv_pair_packed_ex computes, bit for bit, what the two cm_conv_ex calls
 * with those epilogues compute. */
size_t cm_conv_pair_packed_size(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                                uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                                uint32_t kw, uint32_t stride, uint32_t dilation, uint32_t pad_top,
                                uint32_t pad_left, uint32_t out_ch);
int cm_conv_pair_pack(const int16_t *w1, const int16_t *w2, uint32_t batch, uint32_t in_ch,
                      uint32_t in_h, uint32_t in_w, uint32_t mid_ch, uint32_t out_h, uint32_t out_w,
                      uint32_t kh, uint32_t kw, uint32_t stride, uint32_t dilation, uint32_t pad_top,
                      uint32_t pad_left, uint32_t out_ch, void *packed, size_t packed_bytes,
                      hipStream_t stream);
int cm_conv_pair_packed_ex(const int16_t *x, const void *packed, const int16_t *bias1,
                           const int16_t *bias2, int16_t *y, uint32_t batch, uint32_t in_ch,
                           uint32_t in_h, uint32_t in_w, uint32_t mid_ch, uint32_t out_h,
                           uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride,
                           uint32_t dilation, uint32_t pad_top, uint32_t pad_left, uint32_t out_ch,
                           uint32_t act1, const cm_epilogue_t *epi2, hipStream_t stream);

/* A 1x1 convolution (stride 1, no padding, optional bias), its activation
 * (act: 0 none, 1 Relu, 2 Clip(0,6)) and a GlobalAveragePool of every output
 * plane as one launch: y [batch][out_ch] receives what cm_conv_ex (epilogue
 * act) followed by cm_pool (global average) would write, bit for bit, and the
 * convolution's output never reaches memory.  No counterpart in the
 * reference: the scheduler's fusion of a network head (ConvKernel.cpp:171-249
 * then PoolingKernel.cpp:253-266).  x [batch][in_ch][hw], weight
 * [out_ch][in_ch].  cm_conv_gap_supported returns 1 for the shapes the fused
 * kernel takes (hw at most 64, in_ch at most 512), else 0; cm_conv_gap
 * returns CM_ERR_INVALID for the others. */
int cm_conv_gap_supported(uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch);
int cm_conv_gap(const int16_t *x, const int16_t *weight, const int16_t *bias, int16_t *y,
                uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch, uint32_t act,
                hipStream_t stream);

/* cm_matmul_ex for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments and result as cm_matmul_ex
 * without the workspace: its split-K partial sums go to a static 16 MiB
 * device array the library holds on each GPU until the process ends.  A shape
 * whose partials would need more returns CM_ERR_RANGE (launching nothing).
 * Every call on one GPU shares that GPU's array, so calls that overlap in time
 * on one GPU (different streams, a replayed graph beside eager work) race. */
int cm_matmul_noalloc(const int16_t *a, const int16_t *b, int16_t *c, uint32_t n, uint32_t k,
                      uint32_t m, uint32_t batch, uint32_t a_stride, uint32_t b_stride,
                      uint32_t c_stride, const cm_epilogue_t *epi, hipStream_t stream);

/* Default workspace for cm_matmul / cm_matmul_at / cm_conv / cm_run_* (which
 * take none), like cm_set_stream for the stream: device memory the caller
 * allocated and keeps alive while calls may use it.  NULL / 0 = none (the
 * default). */
int cm_set_workspace(void *workspace, size_t bytes);

/* ------------------------------------------------------------------ buffers */

/* Mirrors inference_buf_t (bench_src/inference.h:12-21): an owning allocation
 * or a non-owning view at an element offset.  `host` is the CPU-side mirror
 * (pinned; the reference's `virt`), `dev` the device address (the reference's
 * `phys`).  Transfers happen only in the two sync calls. */
typedef struct cm_buf {
    int16_t *host;
    int16_t *dev;
    uint32_t count;
    uint8_t is_owner;
} cm_buf_t;

int cm_buf_pool_init(void);                       /* inference_buf_pool_init */
void cm_buf_pool_deinit(void);                    /* inference_buf_pool_deinit */
cm_buf_t *cm_buf_alloc(uint32_t n_elem);          /* inference_buf_alloc; NULL on failure */
void cm_buf_free(cm_buf_t *buf);                  /* inference_buf_free (views: no-op) */
int16_t *cm_buf_ptr(cm_buf_t *buf);               /* inference_buf_ptr: host mirror */
int16_t *cm_buf_dev(cm_buf_t *buf);               /* inference_buf_phys: device address */
uint32_t cm_buf_count(const cm_buf_t *buf);       /* inference_buf_count */
void cm_buf_init_view(cm_buf_t *view, cm_buf_t *base, uint32_t offset_elems,
                      uint32_t count_elems);      /* inference_buf_init_view */
int cm_buf_sync_to_device(cm_buf_t *buf);         /* host -> device, stream-ordered */
int cm_buf_sync_from_device(cm_buf_t *buf);       /* device -> host, then waits */

/* Buffer-level helpers with the generated run_* signatures (_source.py:198-421).
 * They enqueue on the stream set by cm_set_stream.  Unlike the reference's void
 * helpers they check every element the call touches against each buffer's
 * count and return CM_ERR_RANGE (nothing launched) when a buffer is too small. */
int cm_run_op(cm_buf_t *a, cm_buf_t *b, cm_buf_t *c, uint32_t size, uint32_t op,
              uint32_t outer, uint32_t a_inc, uint32_t b_inc);
int cm_run_matmul(cm_buf_t *a, cm_buf_t *b, cm_buf_t *c, uint32_t n, uint32_t k, uint32_t m,
                  uint32_t batch, uint32_t a_stride, uint32_t b_stride, uint32_t c_stride);
int cm_run_matmul_at(cm_buf_t *a, uint32_t a_off, cm_buf_t *b, uint32_t b_off, cm_buf_t *c,
                     uint32_t c_off, uint32_t n, uint32_t k, uint32_t m, uint32_t batch,
                     uint32_t a_stride, uint32_t b_stride, uint32_t c_stride);
int cm_run_conv(cm_buf_t *x, cm_buf_t *weight, cm_buf_t *bias, cm_buf_t *y, uint32_t batch,
                uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h,
                uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h, uint32_t stride_w,
                uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left,
                uint32_t has_bias, uint32_t is_depthwise);
int cm_run_pool(cm_buf_t *x, cm_buf_t *y, uint32_t batch, uint32_t channels, uint32_t in_h,
                uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t pool_h, uint32_t pool_w,
                uint32_t stride_h, uint32_t stride_w, uint32_t pad_top, uint32_t pad_left,
                uint32_t dil_h, uint32_t dil_w, uint32_t pool_type, uint32_t lp_order,
                uint32_t count_include_pad);

/* ------------------------------------------------------------------ runtime */

int cm_set_stream(hipStream_t stream);   /* stream used when a call passes NULL */
hipStream_t cm_get_stream(void);
int cm_sync(hipStream_t stream);         /* wait for all work queued on stream */
const char *cm_last_error(void);
const char *cm_version(void);

/* Self-checks of the two scalar paths that use float arithmetic (no reference
 * counterpart; used by the parity tests).  All run on `stream` and wait.
 *   cm_selftest_div: compares the VectorOP DIV path with exact integer
 *     division for every a and every b in [b_lo, b_lo + b_count) (b as uint16
 *     bit patterns); *mismatches receives the count and *example (may be NULL)
 *     one failing case packed as a<<48 | b<<32 | got<<16 | want (16-bit raw).
 *   cm_selftest_finalize: mode 0 = LP p=2 finaliser over accumulators
 *     lo .. lo+count-1; mode 1 = AVG finaliser over accumulators (lo+i) << 8
 *     with denominator d; *checksum = sum (uint16)out * ((lo+i) | 1) mod 2^64. */
int cm_selftest_div(uint32_t b_lo, uint32_t b_count, uint64_t *mismatches, uint64_t *example,
                    hipStream_t stream);
int cm_selftest_finalize(uint32_t mode, uint32_t lo, uint32_t count, uint32_t d,
                         uint64_t *checksum, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* CORMORANT_AMD_H */
