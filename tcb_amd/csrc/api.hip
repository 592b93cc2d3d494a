// api.hip -- the C-ABI of libtrhip (include/trhip.h): contexts, memory, weight stores, dispatch.
//
// Dispatch mirrors the reference's GPU backend (gpu/backend_quant.go:43-65) and CPU backend
// (tensor/cpu_dtype.go:438-466): K == 0 is the empty sum, M == 1 goes to the decode GEMV, M > 1 to the
// chunked rows kernel; the act-quant operator quantizes x on the device and runs the integer block
// kernels. No entry point throws or aborts; errors come back as status codes with a detail string.
#include "trhip_internal.hpp"

#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

namespace trhip {

int fail(trhip_ctx *ctx, int code, const std::string &msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int hip_fail(trhip_ctx *ctx, hipError_t e, const char *what) {
    int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? TRHIP_ERR_OOM : TRHIP_ERR_HIP;
    return fail(ctx, code, std::string(what) + ": " + hipGetErrorName(e));
}

int launch_check(trhip_ctx *ctx, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ctx, TRHIP_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorName(e));
    return TRHIP_OK;
}

void *workspace(trhip_ctx *ctx, size_t bytes, int *status) {
    *status = TRHIP_OK;
    if (bytes <= ctx->ws_bytes) return ctx->ws;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        *status = fail(ctx, TRHIP_ERR_INVALID, "workspace must be sized by an eager call before graph capture");
        return nullptr;
    }
    // Growing: earlier work on the stream may still read the old buffer.
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { *status = hip_fail(ctx, e, "workspace sync"); return nullptr; }
    if (ctx->ws) (void)hipFree(ctx->ws);
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
    size_t want = bytes < (size_t)(1 << 20) ? (size_t)(1 << 20) : bytes + bytes / 4;
    e = hipMalloc(&ctx->ws, want);
    if (e != hipSuccess) { ctx->ws = nullptr; *status = hip_fail(ctx, e, "workspace alloc"); return nullptr; }
    ctx->ws_bytes = want;
    return ctx->ws;
}

void *workspace2(trhip_ctx *ctx, size_t bytes, int *status) {
    *status = TRHIP_OK;
    if (bytes <= ctx->ws2_bytes) return ctx->ws2;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        *status = fail(ctx, TRHIP_ERR_INVALID, "workspace must be sized by an eager call before graph capture");
        return nullptr;
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { *status = hip_fail(ctx, e, "workspace sync"); return nullptr; }
    if (ctx->ws2) (void)hipFree(ctx->ws2);
    ctx->ws2 = nullptr;
    ctx->ws2_bytes = 0;
    size_t want = bytes < (size_t)(1 << 20) ? (size_t)(1 << 20) : bytes + bytes / 4;
    e = hipMalloc(&ctx->ws2, want);
    if (e != hipSuccess) { ctx->ws2 = nullptr; *status = hip_fail(ctx, e, "workspace alloc"); return nullptr; }
    ctx->ws2_bytes = want;
    return ctx->ws2;
}

__global__ void zero_f32_kernel(float *__restrict__ p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

// Zero n floats with a kernel (safe inside graph capture, unlike a memset node).
int zero_f32(trhip_ctx *ctx, float *p, int64_t n) {
    if (n <= 0) return TRHIP_OK;
    hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, p, n);
    return launch_check(ctx, "zero");
}

}  // namespace trhip

using namespace trhip;

namespace {

thread_local std::string g_noctx_err;

bool bad_dtype(int dt) { return dt < TRHIP_Q8 || dt > TRHIP_Q6K; }

struct DevGuard {  // bind the context's device for the duration of a call (gpu/gpu.go:211-232)
    int prev = -1;
    explicit DevGuard(const trhip_ctx *ctx) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (ctx && prev != ctx->device) (void)hipSetDevice(ctx->device);
    }
    ~DevGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

bool bad_scale16(const uint8_t *p) { return ((p[0] | (p[1] << 8)) & 0x7C00) == 0x7C00; }

}  // namespace

extern "C" {

const char *trhip_strerror(int code) {
    switch (code) {
    case TRHIP_OK: return "ok";
    case TRHIP_ERR_INVALID: return "invalid argument";
    case TRHIP_ERR_OOM: return "out of device memory";
    case TRHIP_ERR_HIP: return "HIP runtime error";
    case TRHIP_ERR_LAUNCH: return "kernel launch failed";
    case TRHIP_ERR_UNSUPPORTED: return "unsupported dtype or shape for this operator";
    case TRHIP_ERR_NO_DEVICE: return "no HIP device";
    case TRHIP_ERR_BAD_SCALE: return "NaN or infinite fp16 scale";
    }
    return "unknown error";
}

const char *trhip_last_error(const trhip_ctx *ctx) { return ctx ? ctx->err.c_str() : g_noctx_err.c_str(); }

int trhip_version(void) { return 1; }

int trhip_device_count(int *count) {
    if (!count) return TRHIP_ERR_INVALID;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    return e == hipSuccess ? TRHIP_OK : TRHIP_ERR_NO_DEVICE;
}

int trhip_init(int device, trhip_ctx **out) {
    if (!out) return TRHIP_ERR_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        g_noctx_err = "no HIP device";
        return TRHIP_ERR_NO_DEVICE;
    }
    if (device < 0 || device >= n) {
        g_noctx_err = "device index out of range";
        return TRHIP_ERR_INVALID;
    }
    trhip_ctx *ctx = new (std::nothrow) trhip_ctx();
    if (!ctx) return TRHIP_ERR_OOM;
    ctx->device = device;
    DevGuard g(ctx);
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        g_noctx_err = std::string("stream create: ") + hipGetErrorName(e);
        delete ctx;
        return TRHIP_ERR_HIP;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) ctx->sm_count = prop.multiProcessorCount;
    *out = ctx;
    return TRHIP_OK;
}

int trhip_destroy(trhip_ctx *ctx) {
    if (!ctx) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->ws2) (void)hipFree(ctx->ws2);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return TRHIP_OK;
}

void *trhip_stream(trhip_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int trhip_alloc(trhip_ctx *ctx, size_t bytes, void **dptr) {
    if (!ctx || !dptr) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    *dptr = nullptr;
    hipError_t e = hipMalloc(dptr, bytes ? bytes : 1);
    if (e != hipSuccess) return hip_fail(ctx, e, "alloc");
    return TRHIP_OK;
}

int trhip_free(trhip_ctx *ctx, void *dptr) {
    if (!ctx) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    if (!dptr) return TRHIP_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = hipFree(dptr);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "free");
}

int trhip_h2d_async(trhip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return TRHIP_ERR_INVALID;
    if (!bytes) return TRHIP_OK;
    DevGuard g(ctx);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "h2d");
}

int trhip_d2h(trhip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    hipError_t e = bytes ? hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream) : hipSuccess;
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "d2h");
}

int trhip_memset_async(trhip_ctx *ctx, void *dst, int value, size_t bytes) {
    if (!ctx || (bytes && !dst)) return TRHIP_ERR_INVALID;
    if (!bytes) return TRHIP_OK;
    DevGuard g(ctx);
    hipError_t e = hipMemsetAsync(dst, value, bytes, ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "memset");
}

int trhip_sync(trhip_ctx *ctx) {
    if (!ctx) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "sync");
}

int trhip_event_create(trhip_ctx *ctx, void **ev) {
    if (!ctx || !ev) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    hipEvent_t e0;
    hipError_t e = hipEventCreate(&e0);
    if (e != hipSuccess) return hip_fail(ctx, e, "event create");
    *ev = (void *)e0;
    return TRHIP_OK;
}

int trhip_event_record(trhip_ctx *ctx, void *ev) {
    if (!ctx || !ev) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    hipError_t e = hipEventRecord((hipEvent_t)ev, ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "event record");
}

int trhip_event_elapsed_ms(void *a, void *b, float *ms) {
    if (!a || !b || !ms) return TRHIP_ERR_INVALID;
    hipError_t e = hipEventSynchronize((hipEvent_t)b);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b);
    return e == hipSuccess ? TRHIP_OK : TRHIP_ERR_HIP;
}

int trhip_event_destroy(void *ev) {
    if (!ev) return TRHIP_ERR_INVALID;
    return hipEventDestroy((hipEvent_t)ev) == hipSuccess ? TRHIP_OK : TRHIP_ERR_HIP;
}

int trhip_graph_begin(trhip_ctx *ctx) {
    if (!ctx) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "graph begin");
}

int trhip_graph_end(trhip_ctx *ctx, void **exec) {
    if (!ctx || !exec) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    *exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (e != hipSuccess) return hip_fail(ctx, e, "graph end");
    hipGraphExec_t ge = nullptr;
    e = hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(ctx, e, "graph instantiate");
    *exec = (void *)ge;
    return TRHIP_OK;
}

int trhip_graph_launch(trhip_ctx *ctx, void *exec) {
    if (!ctx || !exec) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    hipError_t e = hipGraphLaunch((hipGraphExec_t)exec, ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "graph launch");
}

int trhip_graph_destroy(void *exec) {
    if (!exec) return TRHIP_ERR_INVALID;
    return hipGraphExecDestroy((hipGraphExec_t)exec) == hipSuccess ? TRHIP_OK : TRHIP_ERR_HIP;
}

int trhip_check_quant_scales(int dtype, const void *raw, size_t raw_bytes, int64_t *bad_block) {
    if (bad_dtype(dtype) || !bad_block || (raw_bytes && !raw)) return TRHIP_ERR_INVALID;
    const uint8_t *r = static_cast<const uint8_t *>(raw);
    size_t size = (size_t)block_bytes(dtype);
    *bad_block = -1;
    for (size_t b = 0; b * size < raw_bytes; b++) {  // tensor/quant.go:108-128 (a short tail block reads its first bytes)
        const uint8_t *blk = r + b * size;
        size_t left = raw_bytes - b * size;
        bool bad = false;
        if (dtype == TRHIP_Q8 || dtype == TRHIP_Q4) bad = left >= 2 && bad_scale16(blk);
        else if (dtype == TRHIP_Q4K) bad = (left >= 2 && bad_scale16(blk)) || (left >= 4 && bad_scale16(blk + 2));
        else bad = left >= 210 && bad_scale16(blk + 208);
        if (bad) {
            *bad_block = (int64_t)b;
            break;
        }
    }
    return TRHIP_OK;
}

int trhip_wstore_create(trhip_ctx *ctx, int dtype, const void *raw, size_t raw_bytes, int64_t N, int64_t K,
                        trhip_wstore **out) {
    if (!ctx || !out) return TRHIP_ERR_INVALID;
    *out = nullptr;
    if (bad_dtype(dtype)) return fail(ctx, TRHIP_ERR_INVALID, "wstore: unknown dtype");
    if (N < 0 || K < 0 || K % block_elems(dtype) != 0)  // H6692: last axis must be a multiple of the block
        return fail(ctx, TRHIP_ERR_INVALID, "wstore: K must be a non-negative multiple of the block size");
    int64_t nb = K / block_elems(dtype);
    size_t need = (size_t)(N * nb) * (size_t)block_bytes(dtype);
    if (raw_bytes != need || (need && !raw))  // H3035
        return fail(ctx, TRHIP_ERR_INVALID, "wstore: raw size does not match N*K");
    int64_t bad = -1;
    trhip_check_quant_scales(dtype, raw, raw_bytes, &bad);
    if (bad >= 0) return fail(ctx, TRHIP_ERR_BAD_SCALE, "wstore: block " + std::to_string(bad) + " has a NaN/Inf scale (H6686)");
    DevGuard g(ctx);
    trhip_wstore *w = new (std::nothrow) trhip_wstore();
    if (!w) return TRHIP_ERR_OOM;
    w->ctx = ctx;
    w->dtype = dtype;
    w->N = N;
    w->K = K;
    w->nb = nb;
    size_t nblk = (size_t)(N * nb);
    size_t o_qs = 0;
    size_t o_aux = align_up(o_qs + nblk * qs_bytes(dtype), 256);
    size_t o_sc = align_up(o_aux + nblk * aux_bytes(dtype), 256);
    size_t o_d = align_up(o_sc + nblk * sc_bytes(dtype), 256);
    size_t total = align_up(o_d + nblk * d_bytes(dtype), 256);
    hipError_t e = hipMalloc(&w->base, total ? total : 256);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(ctx, e, "wstore alloc");
    }
    w->bytes = total;
    w->qs = w->base + o_qs;
    w->aux = aux_bytes(dtype) ? w->base + o_aux : nullptr;
    w->sc = sc_bytes(dtype) ? w->base + o_sc : nullptr;
    w->d = d_bytes(dtype) ? reinterpret_cast<uint16_t *>(w->base + o_d) : nullptr;
    if (need) {
        uint8_t *stage = nullptr;
        e = hipMallocAsync((void **)&stage, need, ctx->stream);
        if (e == hipSuccess) e = hipMemcpyAsync(stage, raw, need, hipMemcpyHostToDevice, ctx->stream);
        int st = e == hipSuccess ? launch_repack(ctx, w, stage) : hip_fail(ctx, e, "wstore upload");
        if (stage) (void)hipFreeAsync(stage, ctx->stream);
        if (st != TRHIP_OK) {
            (void)hipStreamSynchronize(ctx->stream);
            (void)hipFree(w->base);
            delete w;
            return st;
        }
    }
    *out = w;
    return TRHIP_OK;
}

int trhip_wstore_concat(trhip_ctx *ctx, const trhip_wstore *const *parts, int nparts, trhip_wstore **out) {
    if (!ctx || !out) return TRHIP_ERR_INVALID;
    *out = nullptr;
    if (!parts || nparts < 1) return fail(ctx, TRHIP_ERR_INVALID, "wstore_concat: no parts");
    const trhip_wstore *p0 = parts[0];
    if (!p0) return fail(ctx, TRHIP_ERR_INVALID, "wstore_concat: null part");
    int64_t N = 0;
    for (int i = 0; i < nparts; i++) {
        const trhip_wstore *p = parts[i];
        if (!p || p->ctx != ctx) return fail(ctx, TRHIP_ERR_INVALID, "wstore_concat: part of another context");
        if (p->dtype != p0->dtype || p->K != p0->K)
            return fail(ctx, TRHIP_ERR_INVALID, "wstore_concat: parts differ in dtype or K");
        N += p->N;
    }
    DevGuard g(ctx);
    trhip_wstore *w = new (std::nothrow) trhip_wstore();
    if (!w) return TRHIP_ERR_OOM;
    const int dtype = p0->dtype;
    w->ctx = ctx;
    w->dtype = dtype;
    w->N = N;
    w->K = p0->K;
    w->nb = p0->nb;
    size_t nblk = (size_t)(N * w->nb);
    size_t o_aux = align_up(nblk * qs_bytes(dtype), 256);
    size_t o_sc = align_up(o_aux + nblk * aux_bytes(dtype), 256);
    size_t o_d = align_up(o_sc + nblk * sc_bytes(dtype), 256);
    size_t total = align_up(o_d + nblk * d_bytes(dtype), 256);
    hipError_t e = hipMalloc(&w->base, total ? total : 256);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(ctx, e, "wstore_concat alloc");
    }
    w->bytes = total;
    w->qs = w->base;
    w->aux = aux_bytes(dtype) ? w->base + o_aux : nullptr;
    w->sc = sc_bytes(dtype) ? w->base + o_sc : nullptr;
    w->d = d_bytes(dtype) ? reinterpret_cast<uint16_t *>(w->base + o_d) : nullptr;
    // every plane is row-major over blocks, so the rows of the parts follow each other plane by plane
    size_t at = 0;
    for (int i = 0; i < nparts && e == hipSuccess; i++) {
        const trhip_wstore *p = parts[i];
        const size_t nbk = (size_t)(p->N * p->nb);
        if (nbk == 0) continue;
        e = hipMemcpyAsync(w->qs + at * qs_bytes(dtype), p->qs, nbk * qs_bytes(dtype), hipMemcpyDeviceToDevice, ctx->stream);
        if (e == hipSuccess && aux_bytes(dtype))
            e = hipMemcpyAsync(w->aux + at * aux_bytes(dtype), p->aux, nbk * aux_bytes(dtype), hipMemcpyDeviceToDevice,
                               ctx->stream);
        if (e == hipSuccess && sc_bytes(dtype))
            e = hipMemcpyAsync(w->sc + at * sc_bytes(dtype), p->sc, nbk * sc_bytes(dtype), hipMemcpyDeviceToDevice,
                               ctx->stream);
        if (e == hipSuccess && d_bytes(dtype))
            e = hipMemcpyAsync(reinterpret_cast<uint8_t *>(w->d) + at * d_bytes(dtype), p->d, nbk * d_bytes(dtype),
                               hipMemcpyDeviceToDevice, ctx->stream);
        at += nbk;
    }
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(w->base);
        delete w;
        return hip_fail(ctx, e, "wstore_concat copy");
    }
    *out = w;
    return TRHIP_OK;
}

int trhip_wstore_destroy(trhip_wstore *w) {
    if (!w) return TRHIP_ERR_INVALID;
    DevGuard g(w->ctx);
    (void)hipStreamSynchronize(w->ctx->stream);
    (void)hipFree(w->base);
    delete w;
    return TRHIP_OK;
}

int trhip_wstore_info(const trhip_wstore *w, int *dtype, int64_t *N, int64_t *K, size_t *device_bytes) {
    if (!w) return TRHIP_ERR_INVALID;
    if (dtype) *dtype = w->dtype;
    if (N) *N = w->N;
    if (K) *K = w->K;
    if (device_bytes) *device_bytes = w->bytes;
    return TRHIP_OK;
}

int trhip_wstore_to_raw(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t rows, void *raw_out) {
    if (!ctx || !w || row0 < 0 || rows < 0 || row0 + rows > w->N || (rows && !raw_out))
        return fail(ctx, TRHIP_ERR_INVALID, "to_raw: bad row range");
    size_t bytes = (size_t)(rows * w->nb) * (size_t)block_bytes(w->dtype);
    if (!bytes) return TRHIP_OK;
    DevGuard g(ctx);
    int st = TRHIP_OK;
    uint8_t *stage = static_cast<uint8_t *>(workspace(ctx, bytes, &st));
    if (!stage) return st;
    if ((st = launch_unpack(ctx, w, row0, rows, stage)) != TRHIP_OK) return st;
    return trhip_d2h(ctx, raw_out, stage, bytes);
}

int trhip_gemm_q(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                 int64_t M, int64_t K, int accumulate, int mode) {
    if (!ctx || !w) return TRHIP_ERR_INVALID;
    if (M < 0 || N < 0 || row0 < 0 || row0 + N > w->N || K != w->K)
        return fail(ctx, TRHIP_ERR_INVALID, "gemm_q: shape does not match the store");
    if (mode != TRHIP_MODE_EXACT && mode != TRHIP_MODE_FAST) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q: bad mode");
    if (M == 0 || N == 0) return TRHIP_OK;
    DevGuard g(ctx);
    if (K == 0) {  // empty sum (gpu/backend_quant.go:51-56)
        if (accumulate) return TRHIP_OK;
        return zero_f32(ctx, c, M * N);
    }
    if (!x || !c) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q: null x or c");
    if (M == 1) {
        const float *xa = x;
        if (reinterpret_cast<uintptr_t>(x) % 16 != 0) {  // kernels read x 16 bytes at a time (backend_quant.go:105-109)
            int st = TRHIP_OK;
            float *tmp = static_cast<float *>(workspace(ctx, (size_t)K * sizeof(float), &st));
            if (!tmp) return st;
            hipError_t e = hipMemcpyAsync(tmp, x, (size_t)K * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
            if (e != hipSuccess) return hip_fail(ctx, e, "gemm_q: align x");
            xa = tmp;
        }
        return launch_gemv(ctx, w, row0, N, xa, c, accumulate != 0, mode);
    }
    // fast mode (tolerance) on matrix cores over fixed-point activations: q4_k from M = 5 (up to 4 rows the exact
    // kernel's 4-row tiles are as fast), q6_k from M = 2; q8_0 / q4_0 run exact (their fast kernel measured slower)
    if (mode == TRHIP_MODE_FAST && ((w->dtype == TRHIP_Q4K && M > 4) || (w->dtype == TRHIP_Q6K && M > 1)))
        return launch_gemm_rows_fast(ctx, w, row0, N, x, c, M, accumulate != 0);
    return launch_gemm_rows(ctx, w, row0, N, x, c, M, accumulate != 0);
}

int trhip_swiglu(trhip_ctx *ctx, const float *gu, int64_t M, int64_t I, float *out) {
    if (!ctx) return TRHIP_ERR_INVALID;
    if (M < 0 || I < 0) return fail(ctx, TRHIP_ERR_INVALID, "swiglu: negative size");
    if (M == 0 || I == 0) return TRHIP_OK;
    if (!gu || !out) return fail(ctx, TRHIP_ERR_INVALID, "swiglu: null pointer");
    DevGuard g(ctx);
    return launch_swiglu(ctx, gu, M, I, out);
}

int trhip_gemm_q_swiglu(trhip_ctx *ctx, const trhip_wstore *w, const float *x, float *out, int64_t M, int64_t K,
                        int mode) {
    if (!ctx || !w) return TRHIP_ERR_INVALID;
    if (w->N % 2 != 0) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_swiglu: the store must hold [gate | up] rows");
    if (M < 0 || K != w->K) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_swiglu: shape does not match the store");
    const int64_t I = w->N / 2;
    if (M == 0 || I == 0) return TRHIP_OK;
    if (!x || !out) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_swiglu: null x or out");
    DevGuard g(ctx);
    // fast decode (M = 1, aligned x): the gate fused into the GEMV where its K-across-lanes kernel applies, the same
    // bits as the two steps below
    if (mode == TRHIP_MODE_FAST && M == 1 && K > 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
        const int r = launch_gemv_fast_swiglu(ctx, w, x, out, I);
        if (r != -1) return r;
    }
    int st = TRHIP_OK;
    float *gu = static_cast<float *>(workspace2(ctx, (size_t)(M * w->N) * sizeof(float), &st));
    if (!gu) return st;
    // fast M > 1 on matrix cores (as trhip_gemm_q dispatches it): the gate fused into the K-slice sum
    if (mode == TRHIP_MODE_FAST && K > 0 && ((w->dtype == TRHIP_Q4K && M > 4) || (w->dtype == TRHIP_Q6K && M > 1)))
        return launch_gemm_rows_fast(ctx, w, 0, w->N, x, gu, M, false, out);
    if ((st = trhip_gemm_q(ctx, w, 0, w->N, x, gu, M, K, 0, mode)) != TRHIP_OK) return st;
    return launch_swiglu(ctx, gu, M, I, out);
}

int trhip_quantize_q8(trhip_ctx *ctx, const float *x, int64_t M, int64_t K, int blk, int8_t *q, float *d,
                      int16_t *bs) {
    if (!ctx || M < 0 || K < 0 || (blk != 32 && blk != 256) || K % blk != 0) return TRHIP_ERR_INVALID;
    if (M == 0 || K == 0) return TRHIP_OK;
    if (!x || !q || !d || !bs || reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(ctx, TRHIP_ERR_INVALID, "quantize_q8: pointers");
    DevGuard g(ctx);
    int st = TRHIP_OK;
    uint8_t *bad = static_cast<uint8_t *>(workspace(ctx, (size_t)(M * (K / blk)), &st));
    if (!bad) return st;
    return launch_quantize_q8(ctx, x, M, K, blk, q, d, bs, bad, nullptr);
}

int trhip_gemm_q_actq(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                      int64_t M, int64_t K, int accumulate) {
    if (!ctx || !w) return TRHIP_ERR_INVALID;
    if (w->dtype == TRHIP_Q8) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemm_q_actq: q8 weights are not supported (H6723)");
    if (M < 0 || N < 0 || row0 < 0 || row0 + N > w->N || K != w->K)
        return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_actq: shape does not match the store");
    if (M == 0 || N == 0) return TRHIP_OK;
    DevGuard g(ctx);
    if (K == 0) {
        if (accumulate) return TRHIP_OK;
        return zero_f32(ctx, c, M * N);
    }
    if (!x || !c) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_actq: null x or c");
    int blk = block_elems(w->dtype);
    int64_t nb = K / blk;
    size_t o_q = 0;
    size_t o_d = align_up(o_q + (size_t)(M * K), 256);
    size_t o_bs = align_up(o_d + (size_t)(M * nb) * sizeof(float), 256);
    size_t o_fl = align_up(o_bs + (size_t)(M * (K / 16)) * sizeof(int16_t), 256);
    size_t o_sj = align_up(o_fl + (size_t)(M * nb), 256);
    size_t o_x = align_up(o_sj + (w->dtype == TRHIP_Q4K ? (size_t)(M * nb) * 32 : 0), 256);
    bool copy_x = reinterpret_cast<uintptr_t>(x) % 16 != 0;
    size_t total = o_x + (copy_x ? (size_t)(M * K) * sizeof(float) : 0);
    int st = TRHIP_OK;
    uint8_t *ws = static_cast<uint8_t *>(workspace(ctx, total, &st));
    if (!ws) return st;
    int8_t *q = reinterpret_cast<int8_t *>(ws + o_q);
    float *d = reinterpret_cast<float *>(ws + o_d);
    int16_t *bs = reinterpret_cast<int16_t *>(ws + o_bs);
    uint8_t *bad = ws + o_fl;  // one flag byte per activation block (NaN/Inf present)
    uint16_t *sj = w->dtype == TRHIP_Q4K ? reinterpret_cast<uint16_t *>(ws + o_sj) : nullptr;  // q4_k msum operands
    const float *xa = x;
    if (copy_x) {
        float *tmp = reinterpret_cast<float *>(ws + o_x);
        hipError_t e = hipMemcpyAsync(tmp, x, (size_t)(M * K) * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "gemm_q_actq: align x");
        xa = tmp;
    }
    if ((st = launch_quantize_q8(ctx, xa, M, K, blk, q, d, bs, bad, sj)) != TRHIP_OK) return st;
    return launch_actq(ctx, w, row0, N, xa, c, M, accumulate != 0, q, d, bs, bad, sj);
}

int trhip_open_q(trhip_ctx *ctx, const trhip_wstore *w, int64_t elem_off, int64_t n, float *out) {
    if (!ctx || !w) return TRHIP_ERR_INVALID;
    int be = block_elems(w->dtype);
    if (elem_off < 0 || n < 0 || elem_off % be || n % be || elem_off + n > w->N * w->K)
        return fail(ctx, TRHIP_ERR_INVALID, "open_q: range must be block aligned and inside the store");
    if (n == 0) return TRHIP_OK;
    if (!out) return fail(ctx, TRHIP_ERR_INVALID, "open_q: null out");
    DevGuard g(ctx);
    return launch_dequant(ctx, w, elem_off / be, n / be, out);
}

int trhip_read_probe(trhip_ctx *ctx, const void *p, int64_t bytes) {
    if (!ctx || bytes < 0) return TRHIP_ERR_INVALID;
    if (bytes == 0) return TRHIP_OK;
    if (!p || bytes % 16 || reinterpret_cast<uintptr_t>(p) % 16)
        return fail(ctx, TRHIP_ERR_INVALID, "read_probe: p and bytes must be 16-byte aligned");
    DevGuard g(ctx);
    return launch_read_probe(ctx, p, bytes);
}

int trhip_embedding_q(trhip_ctx *ctx, const trhip_wstore *w, const int64_t *idx, int64_t nidx, float *out) {
    if (!ctx || !w || nidx < 0) return TRHIP_ERR_INVALID;
    if (nidx == 0) return TRHIP_OK;
    if (!idx || !out) return fail(ctx, TRHIP_ERR_INVALID, "embedding_q: null pointer");
    for (int64_t i = 0; i < nidx; i++)  // H3043: index out of range
        if (idx[i] < 0 || idx[i] >= w->N)
            return fail(ctx, TRHIP_ERR_INVALID, "embedding_q: index " + std::to_string(idx[i]) + " out of range (H3043)");
    DevGuard g(ctx);
    int st = TRHIP_OK;
    int64_t *didx = static_cast<int64_t *>(workspace(ctx, (size_t)nidx * sizeof(int64_t), &st));
    if (!didx) return st;
    hipError_t e = hipMemcpyAsync(didx, idx, (size_t)nidx * sizeof(int64_t), hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);  // idx is caller memory, pageable
    if (e != hipSuccess) return hip_fail(ctx, e, "embedding_q: idx upload");
    return launch_embedding(ctx, w, didx, nidx, out, nullptr);
}

}  // extern "C"
