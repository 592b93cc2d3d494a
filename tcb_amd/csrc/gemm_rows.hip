// gemm_rows.hip -- fp32-activation quant matmul for M > 1, bit-identical to TR's CPU order.
//
// tensor/cpu_quant.go:103-147 (quantGemmPanels) and the tile path (:59-82, gemmPart in
// cpu_matmul.go:330-380) both compute, for every output (m, n): for each 256-deep K chunk a fresh
// fused chain from +0 in ascending k (sgemm6x16, cpu_micro_amd64.s:14-64), the chunk results added
// in chunk order into a cleared `part`, then c[m, n] += part.
//
// Mapping: a workgroup owns 16 weight rows; thread (row, lane) walks chunks p = lane, lane + 16, ...
// For each chunk it dequantizes the 256 weights once (exactly as tensor/quant.go does) and advances up
// to kMB activation rows' chains together; chunk results go to LDS and 128 threads then add them in
// chunk order. x is read through the cache from a k-major copy (xt[k][m]) so the kMB activations of
// one k are contiguous.
#include "trhip_internal.hpp"

namespace trhip {
namespace {

constexpr int kRows = 16, kLanes = 16, kMB = 8, kMaxChunks = 64;  // K <= 16384

template <int DT, bool ACC>
__global__ __launch_bounds__(256) void gemm_rows_kernel(const Planes p, const float *__restrict__ xt, float *__restrict__ c,
                                                        int64_t N, int64_t row0, int64_t M, int64_t K, int64_t ldc) {
    __shared__ float part[kRows][kMaxChunks][kMB];
    const int lane = threadIdx.x % kLanes, rl = threadIdx.x / kLanes;
    const int64_t r = (int64_t)blockIdx.x * kRows + rl;
    const int64_t nchunks = (K + 255) / 256;
    for (int64_t m0 = 0; m0 < M; m0 += kMB) {
        const int mb = (int)((M - m0) < kMB ? (M - m0) : kMB);
        if (r < N) {
            for (int64_t pc = lane; pc < nchunks; pc += kLanes) {
                float chain[kMB];
#pragma unroll
                for (int m = 0; m < kMB; m++) chain[m] = 0.0f;
                int64_t k1 = (pc + 1) * 256 < K ? (pc + 1) * 256 : K;
                for (int64_t k = pc * 256; k < k1; k++) {
                    float wv = deq_at<DT>(p, row0 + r, k);
                    const float *xk = xt + k * M + m0;
#pragma unroll
                    for (int m = 0; m < kMB; m++)
                        if (m < mb) chain[m] = fmaf(xk[m], wv, chain[m]);
                }
#pragma unroll
                for (int m = 0; m < kMB; m++) part[rl][pc][m] = chain[m];
            }
        }
        __syncthreads();
        if (threadIdx.x < kRows * kMB) {
            int rr = threadIdx.x / kMB, m = threadIdx.x % kMB;
            int64_t row = (int64_t)blockIdx.x * kRows + rr;
            if (row < N && m < mb) {
                float s = 0.0f;
                for (int64_t pc = 0; pc < nchunks; pc++) s = s + part[rr][pc][m];
                float *o = c + (m0 + m) * ldc + row;
                if (ACC) *o = *o + s;
                else *o = s;
            }
        }
        __syncthreads();
    }
}

__global__ void transpose_kernel(const float *__restrict__ x, float *__restrict__ xt, int64_t M, int64_t K) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M * K) return;
    int64_t m = i / K, k = i % K;
    xt[k * M + m] = x[i];
}

template <int DT>
int run_rows(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *xt, float *c, int64_t M,
             bool acc) {
    dim3 grid((unsigned)((N + kRows - 1) / kRows)), block(256);
    if (acc)
        hipLaunchKernelGGL((gemm_rows_kernel<DT, true>), grid, block, 0, ctx->stream, w->planes(), xt, c, N, row0, M, w->K, N);
    else
        hipLaunchKernelGGL((gemm_rows_kernel<DT, false>), grid, block, 0, ctx->stream, w->planes(), xt, c, N, row0, M, w->K, N);
    return launch_check(ctx, "gemm_rows");
}

}  // namespace

int launch_gemm_rows(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     int64_t M, bool acc) {
    if (N == 0 || M == 0) return TRHIP_OK;
    if ((w->K + 255) / 256 > kMaxChunks) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemm_rows: K > 16384");
    int st = TRHIP_OK;
    float *xt = static_cast<float *>(workspace(ctx, (size_t)(M * w->K) * sizeof(float), &st));
    if (!xt) return st;
    int64_t total = M * w->K;
    hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream, x, xt, M,
                       w->K);
    if ((st = launch_check(ctx, "transpose")) != TRHIP_OK) return st;
    switch (w->dtype) {
    case kQ8: return run_rows<kQ8>(ctx, w, row0, N, xt, c, M, acc);
    case kQ4: return run_rows<kQ4>(ctx, w, row0, N, xt, c, M, acc);
    case kQ4K: return run_rows<kQ4K>(ctx, w, row0, N, xt, c, M, acc);
    case kQ6K: return run_rows<kQ6K>(ctx, w, row0, N, xt, c, M, acc);
    }
    return fail(ctx, TRHIP_ERR_INVALID, "gemm_rows: bad dtype");
}

}  // namespace trhip
