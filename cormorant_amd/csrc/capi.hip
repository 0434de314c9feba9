// capi.hip -- the extern "C" boundary: argument validation, error reporting,
// stream handling and the DMA-buffer mirror of inference_buf_*.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cm_internal.h"

namespace {

thread_local char g_err[512] = "";
hipStream_t g_stream = nullptr;
void* g_ws = nullptr;      // default split-K workspace (cm_set_workspace), caller-owned
size_t g_ws_bytes = 0;
int g_sync_check = -1;   // CM_SYNC_CHECK=1: wait after every launch (fault localisation)

hipStream_t pick(hipStream_t s) { return s ? s : g_stream; }

bool sync_check() {
    if (g_sync_check < 0) {
        const char* e = getenv("CM_SYNC_CHECK");
        g_sync_check = (e && e[0] == '1') ? 1 : 0;
    }
    return g_sync_check == 1;
}

int hip_fail(hipError_t e, const char* what) {
    return cm_set_error(CM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// A run_* call touches elements [off, off + need) of buffer b; it must hold them.
bool fits(const cm_buf_t* b, uint64_t off, uint64_t need, const char* fn, const char* name) {
    if (off + need <= b->count) return true;
    cm_set_error(CM_ERR_RANGE, "%s: buffer %s holds %u elements, the call touches %llu", fn, name,
                 b->count, (unsigned long long)(off + need));
    return false;
}

// add_mode / act in range, add present when used, column adds only for MatMul.
int check_epilogue(const cm_epilogue_t* e, bool column_ok, const char* fn) {
    if (!e) return CM_OK;
    if (e->add_mode > CM_EPI_ADD_COLUMN || (e->add_mode == CM_EPI_ADD_COLUMN && !column_ok))
        return cm_set_error(CM_ERR_INVALID, "%s: unsupported epilogue add_mode %u", fn, e->add_mode);
    if (e->act > CM_EPI_ACT_RELU6)
        return cm_set_error(CM_ERR_INVALID, "%s: unsupported epilogue act %u", fn, e->act);
    if (e->add_mode != CM_EPI_ADD_NONE && !e->add)
        return cm_set_error(CM_ERR_INVALID, "%s: epilogue add_mode %u with null add", fn, e->add_mode);
    return CM_OK;
}

}  // namespace

int cm_set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int cm_check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    if (sync_check()) {
        e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_fail(e, what);
    }
    return CM_OK;
}

extern "C" {

const char* cm_last_error(void) { return g_err; }
const char* cm_version(void) { return "cormorant_amd 0.1 gfx950"; }

int cm_set_stream(hipStream_t stream) {
    g_stream = stream;
    return CM_OK;
}

hipStream_t cm_get_stream(void) { return g_stream; }

int cm_sync(hipStream_t stream) {
    const hipError_t e = hipStreamSynchronize(pick(stream));
    return e == hipSuccess ? CM_OK : hip_fail(e, "cm_sync");
}

// ---------------------------------------------------------------- kernels --

int cm_vectorop(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size, uint32_t op,
                uint32_t outer, uint32_t a_inc, uint32_t b_inc, hipStream_t stream) {
    if (size == 0 || outer == 0) return CM_OK;
    if (!a || !c) return cm_set_error(CM_ERR_INVALID, "vectorop: null a or c");
    if (op < CM_VECTOROP_RELU && !b) return cm_set_error(CM_ERR_INVALID, "vectorop: null b for binary op %u", op);
    return cm_vectorop_launch(a, b, c, size, op, outer, a_inc, b_inc, pick(stream));
}

int cm_set_workspace(void* workspace, size_t bytes) {
    g_ws = bytes ? workspace : nullptr;
    g_ws_bytes = workspace ? bytes : 0u;
    return CM_OK;
}

int cm_matmul_ex(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                 uint32_t m, uint32_t batch, uint32_t a_stride, uint32_t b_stride,
                 uint32_t c_stride, const cm_epilogue_t* epi, void* workspace,
                 size_t workspace_bytes, hipStream_t stream) {
    if (batch == 0 || n == 0 || m == 0) return CM_OK;
    if (!c || (k > 0 && (!a || !b))) return cm_set_error(CM_ERR_INVALID, "matmul: null pointer");
    const int rc = check_epilogue(epi, true, "matmul");
    if (rc) return rc;
    const LaunchCtx lc{pick(stream), workspace_bytes ? workspace : nullptr,
                       workspace ? workspace_bytes : 0u, nullptr};
    return cm_matmul_launch(a, b, c, n, k, m, batch, a_stride, b_stride, c_stride, epi, lc);
}

int cm_matmul(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
              uint32_t m, uint32_t batch, uint32_t a_stride, uint32_t b_stride,
              uint32_t c_stride, hipStream_t stream) {
    return cm_matmul_ex(a, b, c, n, k, m, batch, a_stride, b_stride, c_stride, nullptr, g_ws,
                        g_ws_bytes, stream);
}

size_t cm_matmul_workspace_size(uint32_t n, uint32_t k, uint32_t m, uint32_t batch,
                                uint32_t a_stride, uint32_t b_stride, uint32_t c_stride) {
    if (batch == 0 || n == 0 || m == 0) return 0;
    size_t need = 0;
    static int16_t probe[8] __attribute__((aligned(16)));   // never dereferenced in a dry run
    const LaunchCtx lc{nullptr, nullptr, 0u, &need};
    if (cm_matmul_launch(probe, probe, probe, n, k, m, batch, a_stride, b_stride, c_stride,
                         nullptr, lc) != CM_OK)
        return 0;
    return need;
}

int cm_matmul_at(const int16_t* a, uint32_t a_off, const int16_t* b, uint32_t b_off,
                 int16_t* c, uint32_t c_off, uint32_t n, uint32_t k, uint32_t m,
                 uint32_t batch, uint32_t a_stride, uint32_t b_stride, uint32_t c_stride,
                 hipStream_t stream) {
    if (!a || !b || !c) return cm_set_error(CM_ERR_INVALID, "matmul_at: null pointer");
    return cm_matmul(a + a_off, b + b_off, c + c_off, n, k, m, batch, a_stride, b_stride,
                     c_stride, stream);
}

int cm_conv_ex(const int16_t* x, const int16_t* weight, const int16_t* bias, int16_t* y,
               uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
               uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
               uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
               uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise,
               const cm_epilogue_t* epi, void* workspace, size_t workspace_bytes,
               hipStream_t stream) {
    if ((uint64_t)batch * out_ch * out_h * out_w == 0) return CM_OK;
    if (!x || !weight || !y) return cm_set_error(CM_ERR_INVALID, "conv: null x, weight or y");
    if (has_bias && !bias) return cm_set_error(CM_ERR_INVALID, "conv: has_bias with null bias");
    if (is_depthwise && out_ch > in_ch)
        return cm_set_error(CM_ERR_INVALID, "conv: depthwise needs out_ch (%u) <= in_ch (%u)", out_ch, in_ch);
    const int rc = check_epilogue(epi, false, "conv");
    if (rc) return rc;
    const LaunchCtx lc{pick(stream), workspace_bytes ? workspace : nullptr,
                       workspace ? workspace_bytes : 0u, nullptr};
    return cm_conv_launch(x, weight, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh,
                          kw, stride_h, stride_w, dilation_h, dilation_w, pad_top, pad_left,
                          has_bias, is_depthwise, epi, lc);
}

int cm_conv(const int16_t* x, const int16_t* weight, const int16_t* bias, int16_t* y,
            uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
            uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
            uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
            uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, hipStream_t stream) {
    return cm_conv_ex(x, weight, bias, y, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                      stride_h, stride_w, dilation_h, dilation_w, pad_top, pad_left, has_bias,
                      is_depthwise, nullptr, g_ws, g_ws_bytes, stream);
}

size_t cm_conv_workspace_size(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                              uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                              uint32_t kw, uint32_t stride_h, uint32_t stride_w,
                              uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                              uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise) {
    if ((uint64_t)batch * out_ch * out_h * out_w == 0) return 0;
    size_t need = 0;
    static int16_t probe[8] __attribute__((aligned(16)));   // never dereferenced in a dry run
    const LaunchCtx lc{nullptr, nullptr, 0u, &need};
    if (cm_conv_launch(probe, probe, has_bias ? probe : nullptr, probe, batch, in_ch, in_h, in_w,
                       out_ch, out_h, out_w, kh, kw, stride_h, stride_w, dilation_h, dilation_w,
                       pad_top, pad_left, has_bias, is_depthwise, nullptr, lc) != CM_OK)
        return 0;
    return need;
}

size_t cm_conv_packed_size(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                           uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                           uint32_t kw, uint32_t stride_h, uint32_t stride_w,
                           uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                           uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise) {
    (void)has_bias;
    if ((uint64_t)batch * out_ch * out_h * out_w == 0) return 0;
    return cm_conv_packed_bytes(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h,
                                stride_w, dilation_h, dilation_w, pad_top, pad_left, is_depthwise);
}

int cm_conv_pack(const int16_t* weight, uint32_t batch, uint32_t in_ch, uint32_t in_h,
                 uint32_t in_w, uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh,
                 uint32_t kw, uint32_t stride_h, uint32_t stride_w, uint32_t dilation_h,
                 uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left, uint32_t has_bias,
                 uint32_t is_depthwise, void* packed, size_t packed_bytes, hipStream_t stream) {
    if (!weight || !packed) return cm_set_error(CM_ERR_INVALID, "conv pack: null weight or packed");
    if (cm_conv_packed_size(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h,
                            stride_w, dilation_h, dilation_w, pad_top, pad_left, has_bias,
                            is_depthwise) == 0)
        return cm_set_error(CM_ERR_INVALID, "conv pack: the shape does not take the patch-GEMM path");
    return cm_conv_pgemm_pack(weight, batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw,
                              stride_h, stride_w, dilation_h, dilation_w, pad_top, pad_left, packed,
                              packed_bytes, pick(stream));
}

int cm_conv_packed_ex(const int16_t* x, const void* packed, const int16_t* bias, int16_t* y,
                      uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                      uint32_t out_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                      uint32_t stride_h, uint32_t stride_w, uint32_t dilation_h,
                      uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left,
                      uint32_t has_bias, uint32_t is_depthwise, const cm_epilogue_t* epi,
                      hipStream_t stream) {
    if ((uint64_t)batch * out_ch * out_h * out_w == 0) return CM_OK;
    if (!x || !packed || !y) return cm_set_error(CM_ERR_INVALID, "conv packed: null x, packed or y");
    if (has_bias && !bias) return cm_set_error(CM_ERR_INVALID, "conv packed: has_bias with null bias");
    const int rc = check_epilogue(epi, false, "conv");
    if (rc) return rc;
    if (cm_conv_packed_size(batch, in_ch, in_h, in_w, out_ch, out_h, out_w, kh, kw, stride_h,
                            stride_w, dilation_h, dilation_w, pad_top, pad_left, has_bias,
                            is_depthwise) == 0)
        return cm_set_error(CM_ERR_INVALID, "conv packed: the shape does not take the patch-GEMM path");
    return cm_conv_pgemm_run_packed(x, packed, has_bias ? bias : nullptr, y, batch, in_ch, in_h, in_w,
                                    out_ch, out_h, out_w, kh, kw, stride_h, stride_w, dilation_h,
                                    dilation_w, pad_top, pad_left, epi, pick(stream));
}

size_t cm_conv_pair_packed_size(uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w,
                                uint32_t mid_ch, uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw,
                                uint32_t stride, uint32_t dilation, uint32_t pad_top, uint32_t pad_left,
                                uint32_t out_ch) {
    if ((uint64_t)batch * mid_ch * out_ch * out_h * out_w == 0 || kh * kw < 2) return 0;
    return cm_conv_pair_pgemm_bytes(batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride,
                                     dilation, pad_top, pad_left, out_ch);
}

int cm_conv_pair_pack(const int16_t* w1, const int16_t* w2, uint32_t batch, uint32_t in_ch,
                      uint32_t in_h, uint32_t in_w, uint32_t mid_ch, uint32_t out_h, uint32_t out_w,
                      uint32_t kh, uint32_t kw, uint32_t stride, uint32_t dilation, uint32_t pad_top,
                      uint32_t pad_left, uint32_t out_ch, void* packed, size_t packed_bytes,
                      hipStream_t stream) {
    if (!w1 || !w2 || !packed) return cm_set_error(CM_ERR_INVALID, "conv pair pack: null weights or packed");
    if (cm_conv_pair_packed_size(batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride, dilation,
                                 pad_top, pad_left, out_ch) == 0)
        return cm_set_error(CM_ERR_INVALID, "conv pair pack: the shapes do not take the pair path");
    return cm_conv_pair_pgemm_pack(w1, w2, batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride,
                             dilation, pad_top, pad_left, out_ch, packed, packed_bytes, pick(stream));
}

int cm_conv_pair_packed_ex(const int16_t* x, const void* packed, const int16_t* bias1,
                           const int16_t* bias2, int16_t* y, uint32_t batch, uint32_t in_ch,
                           uint32_t in_h, uint32_t in_w, uint32_t mid_ch, uint32_t out_h,
                           uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride,
                           uint32_t dilation, uint32_t pad_top, uint32_t pad_left, uint32_t out_ch,
                           uint32_t act1, const cm_epilogue_t* epi2, hipStream_t stream) {
    if ((uint64_t)batch * out_ch * out_h * out_w == 0) return CM_OK;
    if (!x || !packed || !y) return cm_set_error(CM_ERR_INVALID, "conv pair: null x, packed or y");
    if (act1 > 2u) return cm_set_error(CM_ERR_INVALID, "conv pair: act1 %u (0 none, 1 Relu, 2 Clip(0,6))", act1);
    const int rc = check_epilogue(epi2, false, "conv pair");
    if (rc) return rc;
    if (cm_conv_pair_packed_size(batch, in_ch, in_h, in_w, mid_ch, out_h, out_w, kh, kw, stride, dilation,
                                 pad_top, pad_left, out_ch) == 0)
        return cm_set_error(CM_ERR_INVALID, "conv pair: the shapes do not take the pair path");
    return cm_conv_pair_pgemm_run(x, packed, bias1, bias2, y, batch, in_ch, in_h, in_w, mid_ch, out_h,
                                   out_w, kh, kw, stride, dilation, pad_top, pad_left, out_ch, act1, epi2,
                                   pick(stream));
}

int cm_conv_gap_supported(uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch) {
    return cm_conv_gap_fits(batch, in_ch, hw, out_ch) ? 1 : 0;
}

int cm_conv_gap(const int16_t* x, const int16_t* weight, const int16_t* bias, int16_t* y,
                uint32_t batch, uint32_t in_ch, uint32_t hw, uint32_t out_ch, uint32_t act,
                hipStream_t stream) {
    if ((uint64_t)batch * out_ch == 0) return CM_OK;
    if (!x || !weight || !y) return cm_set_error(CM_ERR_INVALID, "conv gap: null x, weight or y");
    if (act > 2u) return cm_set_error(CM_ERR_INVALID, "conv gap: act %u (0 none, 1 Relu, 2 Clip(0,6))", act);
    if (!cm_conv_gap_fits(batch, in_ch, hw, out_ch))
        return cm_set_error(CM_ERR_INVALID, "conv gap: %u channels of %u pixels are outside the fused kernel's "
                            "range (in_ch 1-512, hw 1-64)", in_ch, hw);
    return cm_conv_gap_launch(x, weight, bias, y, batch, in_ch, hw, out_ch, act, pick(stream));
}

int cm_pool(const int16_t* x, int16_t* y, uint32_t batch, uint32_t channels, uint32_t in_h,
            uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t pool_h, uint32_t pool_w,
            uint32_t stride_h, uint32_t stride_w, uint32_t pad_top, uint32_t pad_left,
            uint32_t dil_h, uint32_t dil_w, uint32_t pool_type, uint32_t lp_order,
            uint32_t count_include_pad, hipStream_t stream) {
    if ((uint64_t)batch * channels * out_h * out_w == 0) return CM_OK;
    if (!x || !y) return cm_set_error(CM_ERR_INVALID, "pool: null x or y");
    return cm_pool_launch(x, y, batch, channels, in_h, in_w, out_h, out_w, pool_h, pool_w,
                          stride_h, stride_w, pad_top, pad_left, dil_h, dil_w, pool_type,
                          lp_order, count_include_pad, pick(stream));
}

// ---------------------------------------------------------------- buffers --

int cm_buf_pool_init(void) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "cm_buf_pool_init");
    if (n < 1) return cm_set_error(CM_ERR_HIP, "cm_buf_pool_init: no GPU");
    return CM_OK;
}

void cm_buf_pool_deinit(void) {}

cm_buf_t* cm_buf_alloc(uint32_t n_elem) {
    cm_buf_t* b = (cm_buf_t*)calloc(1, sizeof(cm_buf_t));
    if (!b) { cm_set_error(CM_ERR_NOMEM, "cm_buf_alloc: out of host memory"); return nullptr; }
    const size_t bytes = (size_t)(n_elem ? n_elem : 1) * sizeof(int16_t);
    hipError_t e = hipMalloc((void**)&b->dev, bytes);
    if (e != hipSuccess) { hip_fail(e, "cm_buf_alloc(device)"); free(b); return nullptr; }
    e = hipHostMalloc((void**)&b->host, bytes, hipHostMallocDefault);
    if (e != hipSuccess) { hip_fail(e, "cm_buf_alloc(host)"); (void)hipFree(b->dev); free(b); return nullptr; }
    memset(b->host, 0, bytes);
    e = hipMemset(b->dev, 0, bytes);
    if (e != hipSuccess) {
        hip_fail(e, "cm_buf_alloc(memset)");
        (void)hipHostFree(b->host); (void)hipFree(b->dev); free(b);
        return nullptr;
    }
    b->count = n_elem;
    b->is_owner = 1;
    return b;
}

void cm_buf_free(cm_buf_t* b) {
    if (!b || !b->is_owner) return;
    (void)hipHostFree(b->host);
    (void)hipFree(b->dev);
    free(b);
}

int16_t* cm_buf_ptr(cm_buf_t* b) { return b ? b->host : nullptr; }
int16_t* cm_buf_dev(cm_buf_t* b) { return b ? b->dev : nullptr; }
uint32_t cm_buf_count(const cm_buf_t* b) { return b ? b->count : 0u; }

void cm_buf_init_view(cm_buf_t* view, cm_buf_t* base, uint32_t offset_elems, uint32_t count_elems) {
    if (!view || !base) return;
    view->host = base->host + offset_elems;
    view->dev = base->dev + offset_elems;
    view->count = count_elems;
    view->is_owner = 0;
}

int cm_buf_sync_to_device(cm_buf_t* b) {
    if (!b) return cm_set_error(CM_ERR_INVALID, "sync_to_device: null buffer");
    if (b->count == 0) return CM_OK;
    const hipError_t e = hipMemcpyAsync(b->dev, b->host, (size_t)b->count * 2,
                                        hipMemcpyHostToDevice, g_stream);
    return e == hipSuccess ? CM_OK : hip_fail(e, "sync_to_device");
}

int cm_buf_sync_from_device(cm_buf_t* b) {
    if (!b) return cm_set_error(CM_ERR_INVALID, "sync_from_device: null buffer");
    if (b->count) {
        hipError_t e = hipMemcpyAsync(b->host, b->dev, (size_t)b->count * 2,
                                      hipMemcpyDeviceToHost, g_stream);
        if (e != hipSuccess) return hip_fail(e, "sync_from_device");
    }
    const hipError_t e = hipStreamSynchronize(g_stream);
    return e == hipSuccess ? CM_OK : hip_fail(e, "sync_from_device(wait)");
}

int cm_run_op(cm_buf_t* a, cm_buf_t* b, cm_buf_t* c, uint32_t size, uint32_t op,
              uint32_t outer, uint32_t a_inc, uint32_t b_inc) {
    if (!a || !c || (op < CM_OP_RELU && !b)) return cm_set_error(CM_ERR_INVALID, "run_op: null buffer");
    if (size && outer) {
        const uint64_t o = outer - 1ull;
        if (!fits(a, 0, o * a_inc + size, "run_op", "a") ||
            (op < CM_OP_RELU && !fits(b, 0, o * b_inc + size, "run_op", "b")) ||
            !fits(c, 0, o * ((uint64_t)a_inc + b_inc) + size, "run_op", "c"))
            return CM_ERR_RANGE;
    }
    return cm_vectorop(a->dev, b ? b->dev : nullptr, c->dev, size, op, outer, a_inc, b_inc, nullptr);
}

int cm_run_matmul_at(cm_buf_t* a, uint32_t a_off, cm_buf_t* b, uint32_t b_off, cm_buf_t* c,
                     uint32_t c_off, uint32_t n, uint32_t k, uint32_t m, uint32_t batch,
                     uint32_t a_stride, uint32_t b_stride, uint32_t c_stride) {
    if (!a || !b || !c) return cm_set_error(CM_ERR_INVALID, "run_matmul: null buffer");
    if (n && m && batch) {
        const uint64_t o = batch - 1ull;
        if (!fits(a, a_off, o * a_stride + (uint64_t)n * k, "run_matmul", "a") ||
            !fits(b, b_off, o * b_stride + (uint64_t)k * m, "run_matmul", "b") ||
            !fits(c, c_off, o * c_stride + (uint64_t)n * m, "run_matmul", "c"))
            return CM_ERR_RANGE;
    }
    return cm_matmul_at(a->dev, a_off, b->dev, b_off, c->dev, c_off, n, k, m, batch, a_stride,
                        b_stride, c_stride, nullptr);
}

int cm_run_matmul(cm_buf_t* a, cm_buf_t* b, cm_buf_t* c, uint32_t n, uint32_t k, uint32_t m,
                  uint32_t batch, uint32_t a_stride, uint32_t b_stride, uint32_t c_stride) {
    return cm_run_matmul_at(a, 0, b, 0, c, 0, n, k, m, batch, a_stride, b_stride, c_stride);
}

int cm_run_conv(cm_buf_t* x, cm_buf_t* weight, cm_buf_t* bias, cm_buf_t* y, uint32_t batch,
                uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch, uint32_t out_h,
                uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h, uint32_t stride_w,
                uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top, uint32_t pad_left,
                uint32_t has_bias, uint32_t is_depthwise) {
    if (!x || !weight || !y || (has_bias && !bias))
        return cm_set_error(CM_ERR_INVALID, "run_conv: null buffer");
    const uint64_t ny = (uint64_t)batch * out_ch * out_h * out_w;
    if (ny && (!fits(x, 0, (uint64_t)batch * in_ch * in_h * in_w, "run_conv", "x") ||
               !fits(weight, 0, (uint64_t)out_ch * (is_depthwise ? 1u : in_ch) * kh * kw,
                     "run_conv", "weight") ||
               (has_bias && !fits(bias, 0, out_ch, "run_conv", "bias")) ||
               !fits(y, 0, ny, "run_conv", "y")))
        return CM_ERR_RANGE;
    return cm_conv(x->dev, weight->dev, bias ? bias->dev : nullptr, y->dev, batch, in_ch, in_h,
                   in_w, out_ch, out_h, out_w, kh, kw, stride_h, stride_w, dilation_h,
                   dilation_w, pad_top, pad_left, has_bias, is_depthwise, nullptr);
}

int cm_run_pool(cm_buf_t* x, cm_buf_t* y, uint32_t batch, uint32_t channels, uint32_t in_h,
                uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t pool_h, uint32_t pool_w,
                uint32_t stride_h, uint32_t stride_w, uint32_t pad_top, uint32_t pad_left,
                uint32_t dil_h, uint32_t dil_w, uint32_t pool_type, uint32_t lp_order,
                uint32_t count_include_pad) {
    if (!x || !y) return cm_set_error(CM_ERR_INVALID, "run_pool: null buffer");
    const uint64_t ny = (uint64_t)batch * channels * out_h * out_w;
    if (ny && (!fits(x, 0, (uint64_t)batch * channels * in_h * in_w, "run_pool", "x") ||
               !fits(y, 0, ny, "run_pool", "y")))
        return CM_ERR_RANGE;
    return cm_pool(x->dev, y->dev, batch, channels, in_h, in_w, out_h, out_w, pool_h, pool_w,
                   stride_h, stride_w, pad_top, pad_left, dil_h, dil_w, pool_type, lp_order,
                   count_include_pad, nullptr);
}

// -------------------------------------------------------------- self-tests --

int cm_selftest_div(uint32_t b_lo, uint32_t b_count, uint64_t* mismatches, uint64_t* example,
                    hipStream_t stream) {
    if (!mismatches) return cm_set_error(CM_ERR_INVALID, "selftest_div: null output");
    if (b_lo > 0xFFFFu || b_count == 0 || b_count > 0x10000u - b_lo)
        return cm_set_error(CM_ERR_RANGE, "selftest_div: b range outside int16");
    hipStream_t s = pick(stream);
    unsigned long long* d = nullptr;
    hipError_t e = hipMalloc((void**)&d, 2 * sizeof(*d));
    if (e != hipSuccess) return hip_fail(e, "selftest_div");
    int rc = CM_OK;
    e = hipMemsetAsync(d, 0, 2 * sizeof(*d), s);
    if (e != hipSuccess) rc = hip_fail(e, "selftest_div");
    for (uint32_t done = 0; rc == CM_OK && done < b_count; done += 4096) {
        const uint32_t n = (b_count - done) < 4096u ? (b_count - done) : 4096u;
        rc = cm_div_sweep_launch(b_lo + done, n, d, s);
    }
    unsigned long long h[2] = {0, 0};
    if (rc == CM_OK) {
        e = hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "selftest_div");
    }
    (void)hipFree(d);
    *mismatches = h[0];
    if (example) *example = h[1];
    return rc;
}

int cm_selftest_finalize(uint32_t mode, uint32_t lo, uint32_t count, uint32_t d,
                         uint64_t* checksum, hipStream_t stream) {
    if (!checksum) return cm_set_error(CM_ERR_INVALID, "selftest_finalize: null output");
    if (mode > 1) return cm_set_error(CM_ERR_INVALID, "selftest_finalize: mode must be 0 or 1");
    hipStream_t s = pick(stream);
    unsigned long long* dev = nullptr;
    hipError_t e = hipMalloc((void**)&dev, sizeof(*dev));
    if (e != hipSuccess) return hip_fail(e, "selftest_finalize");
    int rc = CM_OK;
    e = hipMemsetAsync(dev, 0, sizeof(*dev), s);
    if (e != hipSuccess) rc = hip_fail(e, "selftest_finalize");
    if (rc == CM_OK && count) rc = cm_finalize_sweep_launch(mode, lo, count, d, dev, s);
    unsigned long long h = 0;
    if (rc == CM_OK) {
        e = hipMemcpyAsync(&h, dev, sizeof(h), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "selftest_finalize");
    }
    (void)hipFree(dev);
    *checksum = h;
    return rc;
}

}  // extern "C"
