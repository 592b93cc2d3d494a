// io16.hip -- 16-bit activations and outputs of the quantized matmul (trhip_gemm_q_typed): the reference reads a
// 16-bit a as float32, computes in float32 and rounds into a 16-bit c once (gpu/backend_quant.go:41-45 through
// gpu/backend_memory.go:41-52, 98-115). These kernels widen x (and, when accumulating, c) exactly and round the
// float32 result, with the conversions of trhip_internal.hpp (h16_to_f32, f32_to_h16).
#include "trhip_internal.hpp"

namespace trhip {
namespace {

// four elements per thread: one 8-byte load and one 16-byte store (or the tail one by one)
__global__ __launch_bounds__(256) void widen16_kernel(const uint16_t *__restrict__ src, float *__restrict__ dst,
                                                      int64_t n, int io) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (i + 4 <= n && (reinterpret_cast<uintptr_t>(src) & 7) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
        const uint2 h = *reinterpret_cast<const uint2 *>(src + i);
        *reinterpret_cast<float4 *>(dst + i) = make_float4(h16_to_f32(h.x & 0xFFFFu, io), h16_to_f32(h.x >> 16, io),
                                                           h16_to_f32(h.y & 0xFFFFu, io), h16_to_f32(h.y >> 16, io));
        return;
    }
    for (int64_t j = i; j < i + 4 && j < n; j++) dst[j] = h16_to_f32(src[j], io);
}

__global__ __launch_bounds__(256) void round16_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst,
                                                      int64_t n, int io) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (i + 4 <= n && (reinterpret_cast<uintptr_t>(src) & 15) == 0 && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
        const float4 v = *reinterpret_cast<const float4 *>(src + i);
        *reinterpret_cast<uint2 *>(dst + i) = make_uint2(f32_to_h16(v.x, io) | (f32_to_h16(v.y, io) << 16),
                                                         f32_to_h16(v.z, io) | (f32_to_h16(v.w, io) << 16));
        return;
    }
    for (int64_t j = i; j < i + 4 && j < n; j++) dst[j] = (uint16_t)f32_to_h16(src[j], io);
}

unsigned grid4(int64_t n) { return (unsigned)((n + 1023) / 1024); }

}  // namespace

int launch_widen16(trhip_ctx *ctx, const uint16_t *src, float *dst, int64_t n, int io) {
    if (n <= 0) return TRHIP_OK;
    hipLaunchKernelGGL(widen16_kernel, dim3(grid4(n)), dim3(256), 0, ctx->stream, src, dst, n, io);
    return launch_check(ctx, "widen16");
}

int launch_round16(trhip_ctx *ctx, const float *src, uint16_t *dst, int64_t n, int io) {
    if (n <= 0) return TRHIP_OK;
    hipLaunchKernelGGL(round16_kernel, dim3(grid4(n)), dim3(256), 0, ctx->stream, src, dst, n, io);
    return launch_check(ctx, "round16");
}

}  // namespace trhip
