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
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include <unistd.h>

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

bool capturing(trhip_ctx *ctx) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

namespace {
// Grow one of the context's workspace buffers to at least `bytes`. The old buffer is freed at once when no
// instantiated graph of this context exists, else kept on the retired list (a graph's nodes may hold its address).
void *grow(trhip_ctx *ctx, void *&buf, size_t &have, size_t bytes, int *status) {
    *status = TRHIP_OK;
    if (bytes <= have) return buf;
    if (capturing(ctx)) {
        *status = fail(ctx, TRHIP_ERR_INVALID, "workspace must be sized by an eager call before graph capture");
        return nullptr;
    }
    // Growing: earlier work on the stream may still read the old buffer.
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) { *status = hip_fail(ctx, e, "workspace sync"); return nullptr; }
    if (buf) {
        if (ctx->live_graphs > 0) ctx->retired.push_back(buf);
        else (void)hipFree(buf);
    }
    buf = nullptr;
    have = 0;
    size_t want = bytes < (size_t)(1 << 20) ? (size_t)(1 << 20) : bytes + bytes / 4;
    e = hipMalloc(&buf, want);
    if (e != hipSuccess) { buf = nullptr; *status = hip_fail(ctx, e, "workspace alloc"); return nullptr; }
    have = want;
    return buf;
}
}  // namespace

void *workspace(trhip_ctx *ctx, size_t bytes, int *status) { return grow(ctx, ctx->ws, ctx->ws_bytes, bytes, status); }

void *workspace2(trhip_ctx *ctx, size_t bytes, int *status) {
    return grow(ctx, ctx->ws2, ctx->ws2_bytes, bytes, status);
}

void *workspace3(trhip_ctx *ctx, size_t bytes, int *status) {
    return grow(ctx, ctx->ws3, ctx->ws3_bytes, bytes, status);
}

// Raise a kernel's dynamic-LDS cap on the context's device to at least `bytes`. The largest size granted so far is
// kept per (device, kernel): a later call that needs more raises the cap again, one that needs less keeps it.
int allow_dyn_lds(trhip_ctx *ctx, const void *fn, size_t bytes, const char *what) {
    struct Grant {
        int device;
        const void *fn;
        size_t bytes;
    };
    static std::mutex mu;
    static std::vector<Grant> done;
    std::lock_guard<std::mutex> lk(mu);
    Grant *have = nullptr;
    for (auto &d : done)
        if (d.device == ctx->device && d.fn == fn) have = &d;
    if (have && have->bytes >= bytes) return TRHIP_OK;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) return hip_fail(ctx, e, what);
    if (have) have->bytes = bytes;
    else done.push_back(Grant{ctx->device, fn, bytes});
    return TRHIP_OK;
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

// Byte fill: thread i writes bytes [16 i, 16 i + 16) of the range, one 16-byte store where the range is 16-byte
// aligned there, else byte stores.
__global__ void fill_bytes_kernel(uint8_t *__restrict__ p, uint32_t word, int64_t bytes) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, o = 16 * i;
    if (o >= bytes) return;
    uint8_t *q = p + o;
    if (o + 16 <= bytes && reinterpret_cast<uintptr_t>(q) % 16 == 0) {
        *reinterpret_cast<uint4 *>(q) = make_uint4(word, word, word, word);
    } else {
        const int64_t n = bytes - o < 16 ? bytes - o : 16;
        for (int64_t k = 0; k < n; k++) q[k] = (uint8_t)word;
    }
}

// Fill bytes with a value by a kernel (a memset node in a captured graph has given wrong results on replays).
int fill_bytes(trhip_ctx *ctx, void *p, int value, size_t bytes) {
    if (!bytes) return TRHIP_OK;
    const int64_t units = ((int64_t)bytes + 15) / 16;
    const int64_t blocks = (units + 255) / 256;
    if (blocks >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_INVALID, "memset: too large");
    const uint32_t b = (uint32_t)(value & 0xFF), word = b | (b << 8) | (b << 16) | (b << 24);
    hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, static_cast<uint8_t *>(p),
                       word, (int64_t)bytes);
    return launch_check(ctx, "memset");
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

int scratch_dev(trhip_ctx *ctx);  // below, beside the static scratch array

bool bad_scale16(const uint8_t *p) { return ((p[0] | (p[1] << 8)) & 0x7C00) == 0x7C00; }

// The first block in [b0, b1) of raw (raw_bytes long) whose fp16 scale is NaN or Inf, or -1
// (tensor/quant.go:108-128; a short tail block reads its first bytes).
int64_t scan_scales(int dtype, const uint8_t *r, size_t raw_bytes, size_t b0, size_t b1) {
    const size_t size = (size_t)block_bytes(dtype);
    for (size_t b = b0; b < b1; b++) {
        const uint8_t *blk = r + b * size;
        const size_t left = raw_bytes - b * size;
        bool bad = false;
        if (dtype == TRHIP_Q8 || dtype == TRHIP_Q4) bad = left >= 2 && bad_scale16(blk);
        else if (dtype == TRHIP_Q4K) bad = (left >= 2 && bad_scale16(blk)) || (left >= 4 && bad_scale16(blk + 2));
        else bad = left >= 210 && bad_scale16(blk + 208);
        if (bad) return (int64_t)b;
    }
    return -1;
}

// Host work split over threads: fn(t, lo, hi) for T contiguous ranges [lo, hi) that together cover [0, n).
// Range 0 runs on the calling thread, ranges 1..T-1 on a pool of kHostThreads - 1 workers that live until the process
// ends (started on first use; starting threads per call cost 0.2-0.4 ms of a 33 MB store upload). A worker that
// could not be started (std::thread throws on EAGAIN or a process thread limit) leaves its range to the calling
// thread, so no exception leaves this code. One split runs at a time; calls from other threads wait their turn.
constexpr int kHostThreads = 8;
class HostPool {
  public:
    static HostPool &get() {
        static HostPool *pool = new HostPool();  // never destroyed: idle workers may outlive static destructors
        return *pool;
    }
    // fn(t) for t in [0, T): t = 0 on the caller, the others on workers (or the caller where a worker is missing)
    template <class G> void run(int T, G &&fn) {
        if (getpid() != pid_) {  // a forked child has none of the workers: everything on the caller
            for (int t = 0; t < T; t++) fn(t);
            return;
        }
        std::lock_guard<std::mutex> one(run_mu_);
        int nw = 0;
        {
            std::lock_guard<std::mutex> lk(mu_);
            nw = T - 1 < workers_ ? T - 1 : workers_;
            job_ = [&fn](int t) { fn(t); };
            next_ = 1;
            last_ = nw;
            pending_ = nw;
            gen_++;
        }
        cv_.notify_all();
        fn(0);
        for (int t = nw + 1; t < T; t++) fn(t);  // ranges without a worker
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return pending_ == 0; });
        job_ = nullptr;
    }

  private:
    HostPool() : pid_(getpid()) {
        for (int i = 1; i < kHostThreads; i++) {
            try {
                std::thread([this] { loop(); }).detach();
                workers_++;
            } catch (...) {
                break;
            }
        }
    }
    void loop() {
        unsigned seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> lk(mu_);
            cv_.wait(lk, [&] { return gen_ != seen && next_ <= last_; });
            seen = gen_;
            const int t = next_++;
            std::function<void(int)> j = job_;
            lk.unlock();
            j(t);
            lk.lock();
            if (--pending_ == 0) done_.notify_all();
        }
    }
    const pid_t pid_;
    std::mutex run_mu_, mu_;
    std::condition_variable cv_, done_;
    std::function<void(int)> job_;
    unsigned gen_ = 0;
    int next_ = 1, last_ = 0, pending_ = 0, workers_ = 0;
};

template <class F> void for_ranges(size_t n, int T, F &&fn) {
    if (T < 1) T = 1;
    if (T > kHostThreads) T = kHostThreads;
    const size_t part = (n + (size_t)T - 1) / (size_t)T;
    auto range = [&](int t) {
        const size_t lo = part * t < n ? part * t : n, hi = lo + part < n ? lo + part : n;
        if (lo < hi || t == 0) fn(t, lo, hi);
    };
    if (T == 1) {
        range(0);
        return;
    }
    HostPool::get().run(T, range);
}

// Threads for host passes over `bytes` bytes: one below 4 MiB, where starting threads costs more than it saves.
int host_threads(size_t bytes) { return bytes < ((size_t)4 << 20) ? 1 : kHostThreads; }

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
    int st = scratch_dev(ctx);
    if (st == TRHIP_OK) {  // arrival counters start at zero; every kernel that counts leaves them at zero
        const size_t ab = (size_t)trhip_ctx::kArrivalSlots * sizeof(uint32_t);
        e = hipMalloc(reinterpret_cast<void **>(&ctx->arrivals), ab);
        if (e != hipSuccess) {
            ctx->arrivals = nullptr;
            st = hip_fail(ctx, e, "init: arrival counters");
        } else if ((st = zero_f32(ctx, reinterpret_cast<float *>(ctx->arrivals), trhip_ctx::kArrivalSlots)) == TRHIP_OK &&
                   (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) {
            st = hip_fail(ctx, e, "init: arrival counters");
        }
    }
    if (st != TRHIP_OK) {
        g_noctx_err = ctx->err;
        if (ctx->arrivals) (void)hipFree(ctx->arrivals);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return st;
    }
    *out = ctx;
    return TRHIP_OK;
}

int trhip_destroy(trhip_ctx *ctx) {
    if (!ctx) return TRHIP_ERR_INVALID;
    // Stores and graphs keep using the context's stream (and graphs its retired buffers) until they are destroyed.
    if (ctx->live_stores > 0 || ctx->live_graphs > 0)
        return fail(ctx, TRHIP_ERR_INVALID,
                    "destroy: " + std::to_string(ctx->live_stores) + " weight store(s) and " +
                        std::to_string(ctx->live_graphs) + " graph(s) of this context are still alive");
    DevGuard g(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->ws2) (void)hipFree(ctx->ws2);
    if (ctx->ws3) (void)hipFree(ctx->ws3);
    if (ctx->arrivals) (void)hipFree(ctx->arrivals);
    for (void *p : ctx->retired) (void)hipFree(p);
    if (ctx->idx_host) (void)hipHostFree(ctx->idx_host);
    if (ctx->idx_done) (void)hipEventDestroy(ctx->idx_done);
    for (int s = 0; s < trhip_ctx::UP_SLOTS; s++) {
        if (ctx->up_host[s]) (void)hipHostFree(ctx->up_host[s]);
        if (ctx->up_dev[s]) (void)hipFree(ctx->up_dev[s]);
        if (ctx->up_done[s]) (void)hipEventDestroy(ctx->up_done[s]);
    }
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
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "free: not allowed while the stream is captured");
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
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "d2h: waits for the stream; not allowed while it is captured");
    hipError_t e = bytes ? hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream) : hipSuccess;
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "d2h");
}

int trhip_memset_async(trhip_ctx *ctx, void *dst, int value, size_t bytes) {
    if (!ctx || (bytes && !dst)) return TRHIP_ERR_INVALID;
    if (!bytes) return TRHIP_OK;
    DevGuard g(ctx);
    return fill_bytes(ctx, dst, value, bytes);  // a kernel, so that it can be captured like every other call
}

int trhip_sync(trhip_ctx *ctx) {
    if (!ctx) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "sync: not allowed while the stream is captured");
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

}  // extern "C"

// The opaque graph handle: the instantiated graph and the context whose workspace its nodes may address.
struct trhip_graph {
    hipGraphExec_t exec = nullptr;
    trhip_ctx *ctx = nullptr;
};

extern "C" {

int trhip_graph_end(trhip_ctx *ctx, void **exec) {
    if (!ctx || !exec) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    *exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (e != hipSuccess) return hip_fail(ctx, e, "graph end");
    trhip_graph *tg = new (std::nothrow) trhip_graph();
    if (!tg) {
        (void)hipGraphDestroy(graph);
        return fail(ctx, TRHIP_ERR_OOM, "graph end: host allocation");
    }
    e = hipGraphInstantiate(&tg->exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);  // the executable graph keeps its own copy of the nodes
    if (e != hipSuccess) {
        delete tg;
        return hip_fail(ctx, e, "graph instantiate");
    }
    tg->ctx = ctx;
    ctx->live_graphs++;
    *exec = (void *)tg;
    return TRHIP_OK;
}

int trhip_graph_launch(trhip_ctx *ctx, void *exec) {
    if (!ctx || !exec) return TRHIP_ERR_INVALID;
    trhip_graph *tg = static_cast<trhip_graph *>(exec);
    if (tg->ctx != ctx) return fail(ctx, TRHIP_ERR_INVALID, "graph launch: graph of another context");
    DevGuard g(ctx);
    hipError_t e = hipGraphLaunch(tg->exec, ctx->stream);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "graph launch");
}

int trhip_graph_destroy(void *exec) {
    if (!exec) return TRHIP_ERR_INVALID;
    trhip_graph *tg = static_cast<trhip_graph *>(exec);
    trhip_ctx *ctx = tg->ctx;
    DevGuard g(ctx);
    // a replay may still be running on the stream
    hipError_t e = hipStreamSynchronize(ctx->stream);
    hipError_t e2 = hipGraphExecDestroy(tg->exec);
    delete tg;
    if (--ctx->live_graphs == 0) {  // no node can address a retired workspace buffer any more
        for (void *p : ctx->retired) (void)hipFree(p);
        ctx->retired.clear();
    }
    if (e != hipSuccess) return hip_fail(ctx, e, "graph destroy: sync");
    return e2 == hipSuccess ? TRHIP_OK : hip_fail(ctx, e2, "graph destroy");
}

int trhip_set_launch_shape(trhip_ctx *ctx, int knob, int a, int b, int c, int d) {
    if (!ctx) return TRHIP_ERR_INVALID;
    const bool reset = a == 0 && b == 0 && c == 0 && d == 0;
    switch (knob) {
    case TRHIP_KNOB_KL: {  // WAVES, KS, PD, RPW: the instantiated K-across-lanes shapes
        const int code = 1000 * a + 100 * b + 10 * c + d / 8;
        static const int ok[] = {4141, 4142, 4122, 8141, 4242, 4241, 8241, 8441, 4181, 8181, 2181, 4182, 16181, 4441, 8442};
        bool found = reset;
        for (int v : ok) found = found || (v == code && d % 8 == 0);
        if (!found) return fail(ctx, TRHIP_ERR_INVALID, "set_launch_shape: no such K-across-lanes shape");
        ctx->force_kl = reset ? 0 : code;
        return TRHIP_OK;
    }
    case TRHIP_KNOB_FAST_Q4K: {  // D, WAVES, KS, R of the row-sliced q4_k kernel
        const int code = 1000 * a + 100 * b + 10 * c + d;
        static const int ok[] = {2441, 2841, 2421, 2411, 2422, 8421};
        bool found = reset;
        for (int v : ok) found = found || v == code;
        if (!found) return fail(ctx, TRHIP_ERR_INVALID, "set_launch_shape: no such row-sliced q4_k shape");
        ctx->force_fast_q4k = reset ? 0 : code;
        return TRHIP_OK;
    }
    case TRHIP_KNOB_EXACT_ROWS:
        if (!(reset || ((a == 16 || a == 32 || a == 64) && !b && !c && !d)))
            return fail(ctx, TRHIP_ERR_INVALID, "set_launch_shape: exact rows per workgroup must be 16, 32 or 64");
        ctx->force_exact_rows = a;
        return TRHIP_OK;
    case TRHIP_KNOB_EXACT_LANES:
        if (!(reset || ((a == 4 || a == 8 || a == 16) && !b && !c && !d)))
            return fail(ctx, TRHIP_ERR_INVALID, "set_launch_shape: exact lanes per row must be 4, 8 or 16");
        ctx->force_exact_lanes = a;
        return TRHIP_OK;
    case TRHIP_KNOB_ACTQ_TM:
        if (!(reset || ((a == 0 || a == 32 || a == 64) && b >= 0 && b <= 64 && !c && !d)))
            return fail(ctx, TRHIP_ERR_INVALID,
                        "set_launch_shape: act-quant row tile must be 32 or 64 (0: built-in), K slices 0..64");
        ctx->force_actq_tm = a;
        ctx->force_actq_slices = b;
        return TRHIP_OK;
    case TRHIP_KNOB_KL_GRID:
        if (!(reset || (a >= 1 && a <= 65536 && !b && !c && !d)))
            return fail(ctx, TRHIP_ERR_INVALID, "set_launch_shape: K-across-lanes grid takes 1..65536 workgroups");
        ctx->kl_min_wgs = a;
        return TRHIP_OK;
    case TRHIP_KNOB_ROWS16:
        if (!(reset || ((a == 1 || a == 2) && b >= 1 && b <= 64 && !c && !d)))
            return fail(ctx, TRHIP_ERR_INVALID, "set_launch_shape: rows16 takes 1 or 2 tiles per wave and 1..64 slices");
        ctx->force_rows16 = reset ? 0 : 100 * a + b;
        return TRHIP_OK;
    }
    return fail(ctx, TRHIP_ERR_INVALID, "set_launch_shape: unknown knob");
}

int trhip_check_quant_scales(int dtype, const void *raw, size_t raw_bytes, int64_t *bad_block) {
    if (bad_dtype(dtype) || !bad_block || (raw_bytes && !raw)) return TRHIP_ERR_INVALID;
    const uint8_t *r = static_cast<const uint8_t *>(raw);
    const size_t size = (size_t)block_bytes(dtype), nblk = (raw_bytes + size - 1) / size;
    // Ranges are scanned in parallel; the first bad block overall is the first one of the lowest range that has
    // one, the same block a single pass finds.
    int64_t found[kHostThreads];
    for (auto &f : found) f = -1;
    for_ranges(nblk, host_threads(raw_bytes),
               [&](int t, size_t b0, size_t b1) { found[t] = scan_scales(dtype, r, raw_bytes, b0, b1); });
    *bad_block = -1;
    for (int t = 0; t < kHostThreads && *bad_block < 0; t++) *bad_block = found[t];
    return TRHIP_OK;
}

}  // extern "C"

namespace {

// Planes of a new store of N x K (one allocation; layout in trhip_internal.hpp).
int new_store(trhip_ctx *ctx, int dtype, int64_t N, int64_t K, trhip_wstore **out) {
    trhip_wstore *w = new (std::nothrow) trhip_wstore();
    if (!w) return fail(ctx, TRHIP_ERR_OOM, "wstore: host allocation");
    w->ctx = ctx;
    w->dtype = dtype;
    w->N = N;
    w->K = K;
    w->nb = K / block_elems(dtype);
    size_t nblk = (size_t)(N * w->nb);
    size_t o_aux = align_up(nblk * qs_bytes(dtype), 256);
    size_t o_sc = align_up(o_aux + nblk * aux_bytes(dtype), 256);
    size_t o_d = align_up(o_sc + nblk * sc_bytes(dtype), 256);
    size_t total = align_up(o_d + nblk * d_bytes(dtype), 256);
    hipError_t e = hipMalloc(&w->base, total ? total : 256);
    if (e != hipSuccess) {
        delete w;
        return hip_fail(ctx, e, "wstore alloc");
    }
    w->bytes = total;
    w->qs = w->base;
    w->aux = aux_bytes(dtype) ? w->base + o_aux : nullptr;
    w->sc = sc_bytes(dtype) ? w->base + o_sc : nullptr;
    w->d = d_bytes(dtype) ? reinterpret_cast<uint16_t *>(w->base + o_d) : nullptr;
    ctx->live_stores++;
    *out = w;
    return TRHIP_OK;
}

void drop_store(trhip_wstore *w) {
    (void)hipStreamSynchronize(w->ctx->stream);
    (void)hipFree(w->base);
    w->ctx->live_stores--;
    delete w;
}

// Host allocations made by trhip_host_alloc (pinned, page-locked): uploads from inside one need no staging copy.
std::mutex g_pinned_mu;
std::vector<std::pair<uintptr_t, size_t>> g_pinned;

bool inside_pinned(const void *p, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    std::lock_guard<std::mutex> lk(g_pinned_mu);
    for (const auto &r : g_pinned)
        if (a >= r.first && a + bytes <= r.first + r.second) return true;
    return false;
}

constexpr size_t kUpSlot = (size_t)8 << 20;  // bytes per slot of the upload ring (and per upload chunk)

// The context's upload ring: two pinned host buffers and two device staging buffers, made on first use.
int upload_ring(trhip_ctx *ctx) {
    if (ctx->up_slot_bytes) return TRHIP_OK;
    hipError_t e = hipSuccess;
    for (int s = 0; s < trhip_ctx::UP_SLOTS && e == hipSuccess; s++) {
        e = hipHostMalloc(&ctx->up_host[s], kUpSlot, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc(&ctx->up_dev[s], kUpSlot);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->up_done[s], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        for (int s = 0; s < trhip_ctx::UP_SLOTS; s++) {
            if (ctx->up_host[s]) (void)hipHostFree(ctx->up_host[s]);
            if (ctx->up_dev[s]) (void)hipFree(ctx->up_dev[s]);
            if (ctx->up_done[s]) (void)hipEventDestroy(ctx->up_done[s]);
            ctx->up_host[s] = ctx->up_dev[s] = nullptr;
            ctx->up_done[s] = nullptr;
        }
        return hip_fail(ctx, e, "wstore: upload ring");
    }
    ctx->up_slot_bytes = kUpSlot;
    return TRHIP_OK;
}

}  // namespace

extern "C" {

int trhip_host_alloc(trhip_ctx *ctx, size_t bytes, void **hptr) {
    if (!ctx || !hptr) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    *hptr = nullptr;
    hipError_t e = hipHostMalloc(hptr, bytes ? bytes : 1, hipHostMallocDefault);
    if (e != hipSuccess) {
        *hptr = nullptr;
        return hip_fail(ctx, e, "host alloc");
    }
    std::lock_guard<std::mutex> lk(g_pinned_mu);
    g_pinned.emplace_back(reinterpret_cast<uintptr_t>(*hptr), bytes ? bytes : 1);
    return TRHIP_OK;
}

int trhip_host_free(trhip_ctx *ctx, void *hptr) {
    if (!ctx) return TRHIP_ERR_INVALID;
    if (!hptr) return TRHIP_OK;
    DevGuard g(ctx);
    {
        std::lock_guard<std::mutex> lk(g_pinned_mu);
        size_t i = 0;
        for (; i < g_pinned.size() && g_pinned[i].first != reinterpret_cast<uintptr_t>(hptr); i++) {}
        if (i == g_pinned.size()) return fail(ctx, TRHIP_ERR_INVALID, "host free: not from trhip_host_alloc");
        g_pinned.erase(g_pinned.begin() + (ptrdiff_t)i);
    }
    // a copy from it may still be queued
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = hipHostFree(hptr);
    return e == hipSuccess ? TRHIP_OK : hip_fail(ctx, e, "host free");
}

int trhip_wstore_create(trhip_ctx *ctx, int dtype, const void *raw, size_t raw_bytes, int64_t N, int64_t K,
                        trhip_wstore **out) {
    if (!ctx || !out) return TRHIP_ERR_INVALID;
    *out = nullptr;
    if (bad_dtype(dtype)) return fail(ctx, TRHIP_ERR_INVALID, "wstore: unknown dtype");
    if (N < 0 || K < 0 || K % block_elems(dtype) != 0)  // H6692: last axis must be a multiple of the block
        return fail(ctx, TRHIP_ERR_INVALID, "wstore: K must be a non-negative multiple of the block size");
    const int64_t nb = K / block_elems(dtype), bb = block_bytes(dtype);
    size_t need = (size_t)(N * nb) * (size_t)bb;
    if (raw_bytes != need || (need && !raw))  // H3035
        return fail(ctx, TRHIP_ERR_INVALID, "wstore: raw size does not match N*K");
    DevGuard g(ctx);
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "wstore: not allowed while the stream is captured");
    trhip_wstore *w = nullptr;
    int st = new_store(ctx, dtype, N, K, &w);
    if (st != TRHIP_OK) return st;
    if (need && (st = upload_ring(ctx)) != TRHIP_OK) {
        drop_store(w);
        return st;
    }
    // Chunks of whole blocks (a multiple of 8, so every chunk starts 16-byte aligned in each plane) are uploaded
    // and repacked on the device in stream order. The scale gate (H6686) runs on the host beside the DMA:
    // - pageable source: the host copies chunk i into pinned slot i % 2 and scans the copied blocks, with
    //   several threads, while the DMA engine uploads chunk i - 1; a bad block stops before its chunk is sent;
    // - source inside a trhip_host_alloc block: every chunk is queued from where it is at once, and the whole
    //   input is scanned while the DMA runs.
    // Either way the first bad block is the one trhip_check_quant_scales finds, and the store is then dropped.
    const bool pinned = inside_pinned(raw, need);
    const int64_t nblk = N * nb, per = (int64_t)(kUpSlot / (size_t)bb) / 8 * 8;
    const uint8_t *src0 = static_cast<const uint8_t *>(raw);
    int64_t bad = -1;
    for (int64_t b0 = 0, i = 0; b0 < nblk && st == TRHIP_OK && bad < 0; b0 += per, i++) {
        const int s = (int)(i % trhip_ctx::UP_SLOTS);
        const int64_t nbk = nblk - b0 < per ? nblk - b0 : per;
        const size_t bytes = (size_t)(nbk * bb);
        const uint8_t *src = src0 + (size_t)(b0 * bb);
        hipError_t e = hipSuccess;
        if (!pinned) {
            e = hipEventSynchronize(ctx->up_done[s]);  // the slot's previous upload has left it
            if (e == hipSuccess) {
                uint8_t *slot = static_cast<uint8_t *>(ctx->up_host[s]);
                int64_t found[kHostThreads];
                for (auto &f : found) f = -1;
                for_ranges((size_t)nbk, host_threads(bytes), [&](int t, size_t lo, size_t hi) {
                    std::memcpy(slot + lo * (size_t)bb, src + lo * (size_t)bb, (hi - lo) * (size_t)bb);
                    found[t] = scan_scales(dtype, slot, bytes, lo, hi);
                });
                for (int t = 0; t < kHostThreads && bad < 0; t++)
                    if (found[t] >= 0) bad = b0 + found[t];
                if (bad >= 0) break;
                src = slot;
            }
        }
        if (e == hipSuccess) e = hipMemcpyAsync(ctx->up_dev[s], src, bytes, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipEventRecord(ctx->up_done[s], ctx->stream);
        st = e == hipSuccess ? launch_repack(ctx, w, static_cast<const uint8_t *>(ctx->up_dev[s]), b0, nbk)
                             : hip_fail(ctx, e, "wstore upload");
    }
    if (st == TRHIP_OK && pinned) trhip_check_quant_scales(dtype, raw, raw_bytes, &bad);
    if (st == TRHIP_OK && bad >= 0)
        st = fail(ctx, TRHIP_ERR_BAD_SCALE, "wstore: block " + std::to_string(bad) + " has a NaN/Inf scale (H6686)");
    if (st != TRHIP_OK) {
        drop_store(w);
        return st;
    }
    *out = w;
    return TRHIP_OK;
}

int trhip_wstore_create_zero(trhip_ctx *ctx, int dtype, int64_t N, int64_t K, trhip_wstore **out) {
    if (!ctx || !out) return TRHIP_ERR_INVALID;
    *out = nullptr;
    if (bad_dtype(dtype)) return fail(ctx, TRHIP_ERR_INVALID, "wstore_zero: unknown dtype");
    if (N < 0 || K < 0 || K % block_elems(dtype) != 0)
        return fail(ctx, TRHIP_ERR_INVALID, "wstore_zero: K must be a non-negative multiple of the block size");
    DevGuard g(ctx);
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "wstore_zero: not allowed while the stream is captured");
    trhip_wstore *w = nullptr;
    int st = new_store(ctx, dtype, N, K, &w);
    if (st != TRHIP_OK) return st;
    // tensor/quant.go:414-427: every byte 0, except the q4 codes, 0x88 (code 8 opens to (8 - 8) * +0 = +0)
    const size_t nblk = (size_t)(N * w->nb);
    st = fill_bytes(ctx, w->base, 0, w->bytes);
    if (st == TRHIP_OK && dtype == TRHIP_Q4) st = fill_bytes(ctx, w->qs, 0x88, nblk * qs_bytes(dtype));
    if (st != TRHIP_OK) {
        drop_store(w);
        return st;
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
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "wstore_concat: not allowed while the stream is captured");
    const int dtype = p0->dtype;
    trhip_wstore *w = nullptr;
    int st = new_store(ctx, dtype, N, p0->K, &w);
    if (st != TRHIP_OK) return st;
    hipError_t e = hipSuccess;
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
        drop_store(w);
        return hip_fail(ctx, e, "wstore_concat copy");
    }
    *out = w;
    return TRHIP_OK;
}

int trhip_wstore_destroy(trhip_wstore *w) {
    if (!w) return TRHIP_ERR_INVALID;
    DevGuard g(w->ctx);
    if (capturing(w->ctx)) return fail(w->ctx, TRHIP_ERR_INVALID, "wstore_destroy: not allowed while the stream is captured");
    drop_store(w);
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
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "to_raw: waits for the stream; not allowed while it is captured");
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
    // fast mode (tolerance) on matrix cores: q4_k from M = 5 (up to 4 rows the exact kernel's 4-row tiles are as
    // fast), up to 16 rows in one launch over f16 activation pairs, more over fixed-point digits; q4_0 up to 16 rows
    // over f16 activation pairs; q6_k from M = 2; q8_0 and q4_0 beyond 16 rows run exact
    if (mode == TRHIP_MODE_FAST && M <= 16 && ((w->dtype == TRHIP_Q4K && M > 4) || (w->dtype == TRHIP_Q4 && M > 1))) {
        const int r = launch_rows16(ctx, w, row0, N, x, c, M, accumulate != 0);
        if (r != -1) return r;
    }
    if (mode == TRHIP_MODE_FAST && ((w->dtype == TRHIP_Q4K && M > 4) || (w->dtype == TRHIP_Q6K && M > 1)))
        return launch_gemm_rows_fast(ctx, w, row0, N, x, c, M, accumulate != 0);
    return launch_gemm_rows(ctx, w, row0, N, x, c, M, accumulate != 0);
}

int trhip_gemm_q_typed(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, int xtype,
                       void *c, int ctype, int64_t M, int64_t K, int accumulate, int mode) {
    if (!ctx || !w) return TRHIP_ERR_INVALID;
    auto ok_type = [](int t) { return t == TRHIP_F32 || t == TRHIP_F16 || t == TRHIP_BF16; };
    if (!ok_type(xtype) || !ok_type(ctype)) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_typed: bad element type");
    if (xtype == TRHIP_F32 && ctype == TRHIP_F32)
        return trhip_gemm_q(ctx, w, row0, N, static_cast<const float *>(x), static_cast<float *>(c), M, K, accumulate, mode);
    if (M < 0 || N < 0 || row0 < 0 || row0 + N > w->N || K != w->K)
        return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_typed: shape does not match the store");
    if (mode != TRHIP_MODE_EXACT && mode != TRHIP_MODE_FAST) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_typed: bad mode");
    if (M == 0 || N == 0) return TRHIP_OK;
    if (!c || (K != 0 && !x)) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_typed: null x or c");
    DevGuard g(ctx);
    const size_t cb = ctype == TRHIP_F32 ? 4 : 2;
    if (K == 0) {  // empty sum (gpu/backend_quant.go:51-56): c unchanged, or zeroed (+0 in every type)
        if (accumulate) return TRHIP_OK;
        if (ctype == TRHIP_F32) return zero_f32(ctx, static_cast<float *>(c), M * N);
        return fill_bytes(ctx, c, 0, (size_t)(M * N) * cb);
    }
    // 16-bit x and c of one type, read and written directly: the exact decode GEMV; in fast mode the decode GEMV
    // (K across lanes) and the batched decode kernel, where trhip_gemm_q takes them (q4_k from 5 rows, q4_0 from 2,
    // up to 16)
    if (mode == TRHIP_MODE_EXACT && M == 1 && xtype == ctype && reinterpret_cast<uintptr_t>(x) % 8 == 0 &&
        reinterpret_cast<uintptr_t>(c) % 2 == 0)
        return launch_gemv_exact_io(ctx, w, row0, N, x, c, accumulate != 0, xtype);
    if (mode == TRHIP_MODE_FAST && xtype == ctype && reinterpret_cast<uintptr_t>(c) % 2 == 0) {
        if (M == 1 && reinterpret_cast<uintptr_t>(x) % 8 == 0) {
            const int r = launch_gemv_fast_io(ctx, w, row0, N, x, c, accumulate != 0, xtype);
            if (r != -1) return r;
        }
        if (M <= 16 && ((w->dtype == TRHIP_Q4K && M > 4) || (w->dtype == TRHIP_Q4 && M > 1))) {
            const int r = launch_rows16(ctx, w, row0, N, x, c, M, accumulate != 0, nullptr, xtype);
            if (r != -1) return r;
        }
    }
    // otherwise the reference's own sequence (gpu/backend_memory.go:41-52, 98-115): x widened to fp32, c widened when
    // accumulating, the fp32 operator, c rounded once
    const size_t xbytes = xtype == TRHIP_F32 ? 0 : (size_t)(M * K) * sizeof(float);
    const size_t o_c = (xbytes + 255) / 256 * 256;
    const size_t cbytes = ctype == TRHIP_F32 ? 0 : (size_t)(M * N) * sizeof(float);
    int st = TRHIP_OK;
    uint8_t *ws = static_cast<uint8_t *>(workspace3(ctx, o_c + cbytes, &st));
    if (!ws) return st;
    const float *x32 = static_cast<const float *>(x);
    if (xtype != TRHIP_F32) {
        if ((st = launch_widen16(ctx, static_cast<const uint16_t *>(x), reinterpret_cast<float *>(ws), M * K, xtype)))
            return st;
        x32 = reinterpret_cast<const float *>(ws);
    }
    float *c32 = static_cast<float *>(c);
    if (ctype != TRHIP_F32) {
        c32 = reinterpret_cast<float *>(ws + o_c);
        if (accumulate && (st = launch_widen16(ctx, static_cast<const uint16_t *>(c), c32, M * N, ctype))) return st;
    }
    if ((st = trhip_gemm_q(ctx, w, row0, N, x32, c32, M, K, accumulate, mode))) return st;
    if (ctype != TRHIP_F32) return launch_round16(ctx, c32, static_cast<uint16_t *>(c), M * N, ctype);
    return TRHIP_OK;
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
    if (mode == TRHIP_MODE_FAST && K > 0 && w->dtype == TRHIP_Q4K && M > 4 && M <= 16) {
        const int r = launch_rows16(ctx, w, 0, w->N, x, nullptr, M, false, out);
        if (r != -1) return r;
    }
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

}  // extern "C"

namespace {

// Scratch layout of the act-quant operator: q [M][K] int8, d [M][K/blk] fp32, bs [M][K/16] int16, one NaN/Inf flag
// byte per activation block, for q4_k the f16 msum operands [M][K/256][16], and an aligned copy of x when x is not
// 16-byte aligned. When a prefill kernel (q4_k, q6_k) takes the shape (tiles), q, d and the q4_k msum operands are in
// its tiled layout over rows padded to a multiple of 128, and there are no 16-sums.
struct ActqLayout {
    size_t o_q = 0, o_d = 0, o_bs = 0, o_fl = 0, o_sj = 0, o_x = 0, total = 0;
    bool copy_x = false, tiles = false;
};

ActqLayout actq_layout(int dtype, int64_t M, int64_t N, int64_t row0, int64_t K, const float *x) {
    ActqLayout l;
    const int64_t nb = K / block_elems(dtype);
    l.tiles = prefill_tiles_apply(dtype, M, N, row0, K);
    const int64_t Mq = l.tiles ? (M + kPrefillRowPad - 1) / kPrefillRowPad * kPrefillRowPad : M;
    l.o_d = align_up(l.o_q + (size_t)(Mq * K), 256);
    l.o_bs = align_up(l.o_d + (size_t)(Mq * nb) * sizeof(float), 256);
    l.o_fl = align_up(l.o_bs + (l.tiles ? 0 : (size_t)(M * (K / 16)) * sizeof(int16_t)), 256);
    l.o_sj = align_up(l.o_fl + (size_t)(M * nb), 256);
    l.o_x = align_up(l.o_sj + (dtype == TRHIP_Q4K ? (size_t)(Mq * nb) * 32 : 0), 256);
    l.copy_x = reinterpret_cast<uintptr_t>(x) % 16 != 0;
    l.total = l.o_x + (l.copy_x ? (size_t)(M * K) * sizeof(float) : 0);
    return l;
}

// Argument checks shared by both act-quant entry points; 0 = go on, 1 = done (nothing to compute), else a status.
int actq_check(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, int64_t M,
               int64_t K, const char *name, int *status) {
    *status = TRHIP_OK;
    if (w->dtype == TRHIP_Q8)
        return *status = fail(ctx, TRHIP_ERR_UNSUPPORTED, std::string(name) + ": q8 weights are not supported (H6723)"), 2;
    if (M < 0 || N < 0 || row0 < 0 || row0 + N > w->N || K != w->K)
        return *status = fail(ctx, TRHIP_ERR_INVALID, std::string(name) + ": shape does not match the store"), 2;
    if (M == 0 || N == 0) return 1;
    if (K != 0 && (!x || !c)) return *status = fail(ctx, TRHIP_ERR_INVALID, std::string(name) + ": null x or c"), 2;
    return 0;
}

// Quantize x into the scratch `ws` (layout l) and run the integer block kernels.
int actq_run(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, int64_t M,
             int64_t K, int accumulate, uint8_t *ws, const ActqLayout &l, bool fast = false) {
    const int blk = block_elems(w->dtype);
    int8_t *q = reinterpret_cast<int8_t *>(ws + l.o_q);
    float *d = reinterpret_cast<float *>(ws + l.o_d);
    int16_t *bs = reinterpret_cast<int16_t *>(ws + l.o_bs);
    uint8_t *bad = ws + l.o_fl;  // one flag byte per activation block (NaN/Inf present)
    uint16_t *sj = w->dtype == TRHIP_Q4K ? reinterpret_cast<uint16_t *>(ws + l.o_sj) : nullptr;  // q4_k msum operands
    const float *xa = x;
    if (l.copy_x) {
        float *tmp = reinterpret_cast<float *>(ws + l.o_x);
        hipError_t e = hipMemcpyAsync(tmp, x, (size_t)(M * K) * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "gemm_q_actq: align x");
        xa = tmp;
    }
    if (l.tiles) {
        int st = launch_quantize_tiles(ctx, xa, M, K, q, d, sj, bad);
        if (st != TRHIP_OK) return st;
        if (w->dtype == TRHIP_Q6K) return launch_prefill_q6k(ctx, w, row0, N, xa, c, M, accumulate != 0, q, d, bad);
        return launch_prefill_q4k(ctx, w, row0, N, xa, c, M, accumulate != 0, q, d, sj, bad, fast);
    }
    int st = launch_quantize_q8(ctx, xa, M, K, blk, q, d, bs, bad, sj);
    if (st != TRHIP_OK) return st;
    return launch_actq(ctx, w, row0, N, xa, c, M, accumulate != 0, q, d, bs, bad, sj, fast);
}

}  // namespace

// The allocation-free act-quant's scratch (trhip_gemm_q_actq_noalloc): one copy per device, held until the process
// ends. Host code never uses this name as an address: the device address comes from hipGetSymbolAddress, once per
// device, in trhip_init (scratch_dev below).
static __device__ __align__(256) uint8_t scratch[TRHIP_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void *g_scratch_dev[64] = {};  // device address of `scratch` on device i (set by trhip_init with i current)

// The address of `scratch` on the current device ctx->device; looked up on the first context of a device.
int scratch_dev(trhip_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= 64) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "scratch: device index above 63");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[ctx->device]) {
        void *ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return hip_fail(ctx, e != hipSuccess ? e : hipErrorInvalidSymbol, "scratch address");
        g_scratch_dev[ctx->device] = ptr;
    }
    ctx->scratch = static_cast<uint8_t *>(g_scratch_dev[ctx->device]);
    return TRHIP_OK;
}
}  // namespace

extern "C" {

int trhip_gemm_q_actq_mode(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                           int64_t M, int64_t K, int accumulate, int mode) {
    if (!ctx || !w) return TRHIP_ERR_INVALID;
    if (mode != TRHIP_MODE_EXACT && mode != TRHIP_MODE_FAST) return fail(ctx, TRHIP_ERR_INVALID, "gemm_q_actq: unknown mode");
    int st = TRHIP_OK;
    const int r = actq_check(ctx, w, row0, N, x, c, M, K, "gemm_q_actq", &st);
    if (r) return st;
    DevGuard g(ctx);
    if (K == 0) return accumulate ? TRHIP_OK : zero_f32(ctx, c, M * N);
    const ActqLayout l = actq_layout(w->dtype, M, N, row0, K, x);
    uint8_t *ws = static_cast<uint8_t *>(workspace(ctx, l.total, &st));
    if (!ws) return st;
    return actq_run(ctx, w, row0, N, x, c, M, K, accumulate, ws, l, mode == TRHIP_MODE_FAST);
}

int trhip_gemm_q_actq(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                      int64_t M, int64_t K, int accumulate) {
    return trhip_gemm_q_actq_mode(ctx, w, row0, N, x, c, M, K, accumulate, TRHIP_MODE_EXACT);
}

int trhip_gemm_q_actq_noalloc(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x,
                              float *c, int64_t M, int64_t K, int accumulate) {
    if (!ctx || !w) return TRHIP_ERR_INVALID;
    int st = TRHIP_OK;
    const int r = actq_check(ctx, w, row0, N, x, c, M, K, "gemm_q_actq_noalloc", &st);
    if (r) return st;
    if (K != 0) {
        const ActqLayout l = actq_layout(w->dtype, M, N, row0, K, x);
        if (l.total > (size_t)TRHIP_NOALLOC_SCRATCH_BYTES)
            return fail(ctx, TRHIP_ERR_INVALID,
                        "gemm_q_actq_noalloc: M x K needs " + std::to_string(l.total) + " bytes of scratch; the static "
                        "scratch holds " + std::to_string((size_t)TRHIP_NOALLOC_SCRATCH_BYTES) + " (use trhip_gemm_q_actq)");
        if (!ctx->scratch) return fail(ctx, TRHIP_ERR_HIP, "gemm_q_actq_noalloc: no scratch address");
        DevGuard g(ctx);
        return actq_run(ctx, w, row0, N, x, c, M, K, accumulate, ctx->scratch, l);
    }
    DevGuard g(ctx);
    return accumulate ? TRHIP_OK : zero_f32(ctx, c, M * N);
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

int trhip_mfma_probe(trhip_ctx *ctx, int valu_per_mfma, int waves_per_simd, int64_t iters) {
    if (!ctx) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    return launch_mfma_probe(ctx, valu_per_mfma, waves_per_simd, iters);
}

int trhip_prefill_probe(trhip_ctx *ctx, int kind, int64_t M, int64_t N, int64_t K) {
    if (!ctx) return TRHIP_ERR_INVALID;
    DevGuard g(ctx);
    return launch_prefill_probe(ctx, kind, M, N, K);
}

int trhip_embedding_q(trhip_ctx *ctx, const trhip_wstore *w, const int64_t *idx, int64_t nidx, float *out) {
    if (!ctx || !w || nidx < 0) return TRHIP_ERR_INVALID;
    if (nidx == 0) return TRHIP_OK;
    if (!idx || !out) return fail(ctx, TRHIP_ERR_INVALID, "embedding_q: null pointer");
    for (int64_t i = 0; i < nidx; i++)  // H3043: index out of range
        if (idx[i] < 0 || idx[i] >= w->N)
            return fail(ctx, TRHIP_ERR_INVALID, "embedding_q: index " + std::to_string(idx[i]) + " out of range (H3043)");
    DevGuard g(ctx);
    // The indices go through pinned staging owned by the context, so the upload is asynchronous; the staging is
    // rewritten only after the copy that last read it has completed. A captured graph would replay whatever the
    // staging holds then, so host indices are refused during capture.
    if (capturing(ctx))
        return fail(ctx, TRHIP_ERR_INVALID, "embedding_q: host indices cannot be captured into a graph");
    const size_t ib = (size_t)nidx * sizeof(int64_t);
    hipError_t e = hipSuccess;
    if (!ctx->idx_done) e = hipEventCreateWithFlags(&ctx->idx_done, hipEventDisableTiming);
    else e = hipEventSynchronize(ctx->idx_done);
    if (e != hipSuccess) return hip_fail(ctx, e, "embedding_q: staging event");
    if (ib > ctx->idx_host_bytes) {
        if (ctx->idx_host) (void)hipHostFree(ctx->idx_host);
        ctx->idx_host = nullptr;
        ctx->idx_host_bytes = 0;
        const size_t want = ib < 4096 ? 4096 : ib + ib / 4;
        e = hipHostMalloc(&ctx->idx_host, want, hipHostMallocDefault);
        if (e != hipSuccess) {
            ctx->idx_host = nullptr;
            return hip_fail(ctx, e, "embedding_q: staging alloc");
        }
        ctx->idx_host_bytes = want;
    }
    int st = TRHIP_OK;
    int64_t *didx = static_cast<int64_t *>(workspace(ctx, ib, &st));
    if (!didx) return st;
    std::memcpy(ctx->idx_host, idx, ib);
    e = hipMemcpyAsync(didx, ctx->idx_host, ib, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(ctx->idx_done, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "embedding_q: idx upload");
    return launch_embedding(ctx, w, didx, nidx, out, nullptr);
}

}  // extern "C"
