// swiglu.hip -- the SwiGLU epilogue of a merged gate_up projection, bit-identical to TR's CPU path:
// out[m, i] = silu(gu[m, i]) * gu[m, I + i] on the [G | U] row layout of a merged gate_up layer
// (lib/layers.tr:223 swiglu_gate, :240-262 and .split(2)). silu is siluForward
// (tensor/cpu_elementwise_wide.go:101-116 with sigmoidBlock :83-98) and e^x is the AVX2 expVec the
// reference runs for every element (tensor/cpu_vector_amd64.s:13-38): the same operations in the same
// order, with fused multiply-adds exactly where that kernel fuses, and correctly rounded division (silu_ref in
// trhip_internal.hpp, shared with the GEMV that fuses this epilogue).
#include "trhip_internal.hpp"

namespace trhip {
namespace {

__global__ void swiglu_kernel(const float *__restrict__ gu, int64_t M, int64_t I, float *__restrict__ out) {
    const int64_t total = M * I, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
        const int64_t m = t / I, i = t - m * I;
        const float *row = gu + m * 2 * I;
        out[t] = silu_ref(row[i]) * row[I + i];
    }
}

}  // namespace

int launch_swiglu(trhip_ctx *ctx, const float *gu, int64_t M, int64_t I, float *out) {
    const int64_t total = M * I;
    if (total == 0) return TRHIP_OK;
    int64_t blocks = (total + 255) / 256;
    const int64_t cap = (int64_t)(ctx->sm_count > 0 ? ctx->sm_count : 256) * 8;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, gu, M, I, out);
    return launch_check(ctx, "swiglu");
}

}  // namespace trhip
