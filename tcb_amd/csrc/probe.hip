// probe.hip -- streaming-read ceiling of the device (diagnostic, no counterpart in the reference).
//
// The kernel reads a buffer once with the access pattern that measured fastest for one launch on MI355X
// (256 threads, four 16-byte loads per thread issued back to back, one pass over the buffer; deeper or
// grid-stride variants were slower). Timed over a ring of buffers larger than the 256 MB MALL, one launch
// is the practical floor of any kernel that must stream that many bytes from HBM in one launch: the
// GEMV kernels are compared against it. The loaded words are folded into one word per workgroup, which is
// stored only when it equals a fixed pattern, so the loads stay live without memory writes of their own.
#include "trhip_internal.hpp"

namespace trhip {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kReadThreads = 256, kReadPieces = 4;

__global__ __launch_bounds__(kReadThreads) void read_probe_kernel(const u32x4 *__restrict__ p, int64_t n16,
                                                                  uint32_t *__restrict__ sink) {
    u32x4 v[kReadPieces];
#pragma unroll
    for (int u = 0; u < kReadPieces; u++) {
        const int64_t i = ((int64_t)blockIdx.x * kReadPieces + u) * kReadThreads + threadIdx.x;
        v[u] = i < n16 ? p[i] : (u32x4){0u, 0u, 0u, 0u};
    }
    uint32_t s = 0;
#pragma unroll
    for (int u = 0; u < kReadPieces; u++) s ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (s == 0x9E3779B9u) sink[blockIdx.x] = s;
}

}  // namespace

int launch_read_probe(trhip_ctx *ctx, const void *p, int64_t bytes) {
    const int64_t n16 = bytes / 16, per = (int64_t)kReadThreads * kReadPieces;
    const int64_t grid = (n16 + per - 1) / per;
    if (grid >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "read_probe: buffer too large");
    int st = TRHIP_OK;
    uint32_t *sink = static_cast<uint32_t *>(workspace(ctx, (size_t)grid * sizeof(uint32_t), &st));
    if (!sink) return st;
    hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)grid), dim3(kReadThreads), 0, ctx->stream,
                       static_cast<const u32x4 *>(p), n16, sink);
    return launch_check(ctx, "read_probe");
}

}  // namespace trhip
