// probe.hip -- device ceilings the kernels are measured against (diagnostics, no counterpart in the reference):
// the streaming-read ceiling of one launch, and the int8 matrix-core rate with and without VALU work beside it.
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

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Each wave runs `iters` rounds of four independent v_mfma_i32_32x32x32_i8 chains (4 x 65536 int8 ops) and V
// independent v_fma_f32 per MFMA spread over eight float chains, the mix of a prefill kernel's block loop. The
// results are folded into one word stored only when it equals a fixed pattern.
template <int V>
__global__ __launch_bounds__(1024) void mfma_probe_kernel(int64_t iters, uint32_t *__restrict__ sink) {
    const int lane = threadIdx.x & 63;
    const v4i a = (v4i){lane, lane + 1, lane + 2, lane + 3}, b = (v4i){3 * lane, lane ^ 5, 7, lane >> 1};
    v16i acc[4];
#pragma unroll
    for (int t = 0; t < 4; t++) acc[t] = (v16i){0};
    float f[8];
#pragma unroll
    for (int j = 0; j < 8; j++) f[j] = (float)(lane + j);
    const float c1 = 0.999f, c2 = 1e-3f * (float)(threadIdx.x & 7);
    for (int64_t it = 0; it < iters; it++) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[t], 0, 0, 0);
#pragma unroll
            for (int v = 0; v < V; v++) f[(4 * t + v) & 7] = __builtin_fmaf(f[(4 * t + v) & 7], c1, c2);
        }
    }
    uint32_t s = 0;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) s ^= (uint32_t)acc[t][r];
#pragma unroll
    for (int j = 0; j < 8; j++) s ^= __builtin_bit_cast(uint32_t, f[j]);
    if (s == 0x9E3779B9u) sink[blockIdx.x] = s;
}

}  // namespace

int launch_mfma_probe(trhip_ctx *ctx, int valu_per_mfma, int waves_per_simd, int64_t iters) {
    if (iters < 0 || waves_per_simd < 1 || waves_per_simd > 4)
        return fail(ctx, TRHIP_ERR_INVALID, "mfma_probe: waves per SIMD must be 1..4");
    const int cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    int st = TRHIP_OK;
    uint32_t *sink = static_cast<uint32_t *>(workspace(ctx, (size_t)cus * sizeof(uint32_t), &st));
    if (!sink) return st;
    dim3 grid((unsigned)cus), block((unsigned)(256 * waves_per_simd));
    switch (valu_per_mfma) {
    case 0: hipLaunchKernelGGL(mfma_probe_kernel<0>, grid, block, 0, ctx->stream, iters, sink); break;
    case 2: hipLaunchKernelGGL(mfma_probe_kernel<2>, grid, block, 0, ctx->stream, iters, sink); break;
    case 4: hipLaunchKernelGGL(mfma_probe_kernel<4>, grid, block, 0, ctx->stream, iters, sink); break;
    case 6: hipLaunchKernelGGL(mfma_probe_kernel<6>, grid, block, 0, ctx->stream, iters, sink); break;
    case 8: hipLaunchKernelGGL(mfma_probe_kernel<8>, grid, block, 0, ctx->stream, iters, sink); break;
    case 12: hipLaunchKernelGGL(mfma_probe_kernel<12>, grid, block, 0, ctx->stream, iters, sink); break;
    case 16: hipLaunchKernelGGL(mfma_probe_kernel<16>, grid, block, 0, ctx->stream, iters, sink); break;
    default: return fail(ctx, TRHIP_ERR_INVALID, "mfma_probe: VALU per MFMA must be 0, 2, 4, 6, 8, 12 or 16");
    }
    return launch_check(ctx, "mfma_probe");
}

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
