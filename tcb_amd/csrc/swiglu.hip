// swiglu.hip -- the SwiGLU epilogue of a merged gate_up projection, bit-identical to TR's CPU path:
// out[m, i] = silu(gu[m, i]) * gu[m, I + i] on the [G | U] row layout of a merged gate_up layer
// (lib/layers.tr:223 swiglu_gate, :240-262 and .split(2)). silu is siluForward
// (tensor/cpu_elementwise_wide.go:101-116 with sigmoidBlock :83-98) and e^x is the AVX2 expVec the
// reference runs for every element (tensor/cpu_vector_amd64.s:13-38): the same operations in the same
// order, with fused multiply-adds exactly where that kernel fuses, and correctly rounded division.
#include "trhip_internal.hpp"

namespace trhip {
namespace {

__device__ __forceinline__ float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// e^x: clamp to [-104, 89] (NaN takes the lower bound and is put back at the end), n = rne(x log2e),
// r = x - n ln2 in two fused steps (ln2 split high/low), a degree-6 polynomial in fused steps, and 2^n
// applied as 2^(n>>1) * 2^(n - n>>1), so subnormal results and overflow to +Inf come out right.
__device__ __forceinline__ float exp_ref(float x) {
    float x1 = x > -104.0f ? x : -104.0f;
    x1 = x1 < 89.0f ? x1 : 89.0f;
    const float n = __builtin_rintf(x1 * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693359375f, x1);
    r = __builtin_fmaf(-n, -2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    const float z = r * r;
    p = __builtin_fmaf(z, p, r);
    float y = p + 1.0f;
    const int ni = (int)n, h = ni >> 1, l = ni - h;
    y = y * bits_f32((uint32_t)(h + 127) << 23);
    y = y * bits_f32((uint32_t)(l + 127) << 23);
    return x != x ? x : y;
}

}  // namespace

// x sigma(x) with e = e^-|x|: sigma = 1/(1+e) for x >= 0, e/(1+e) otherwise; sigma == 0 gives +0.
__device__ float silu_ref(float x) {
    const float e = exp_ref(-__builtin_fabsf(x));
    const float s = x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    return (s == 0.0f ? 0.0f : x) * s;
}

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
