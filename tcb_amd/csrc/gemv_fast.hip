// gemv_fast.hip -- decode GEMV (M == 1) in factored order: within the tolerance the reference allows a
// device GEMV (|a-b|/(1+|b|) <= 1e-5, 1e-4 for K-quants), not bit-identical to TR's CPU path.
//
// Per 32-element sub-block j with value y = s_j*q - m_j (tensor/quant.go:167-182):
//   sum_e y_e x_e = s_j * (sum_e q_e x_e) - m_j * (sum_e x_e)
// so the inner loop is one convert and one fused multiply-add per weight. The 16-element sums of x are the
// same for every row and are computed once per workgroup into LDS next to x.
//
// Every partial sum is combined in a fixed order inside one workgroup (LDS, then a fixed xor-butterfly),
// with no atomics, so the result depends only on the shape (the reference forbids atomic accumulation on
// this path, gpu/kernel_quant_gemv.go:14-16). q4_k only; the other dtypes use the exact kernel.
#include "trhip_internal.hpp"

#include <cstdio>
#include <cstdlib>

namespace trhip {
namespace {

// ---------------------------------------------------------------- q4_k
// Nibble pairs to floats: a byte holding 0..15, read as an OCP FP8 E4M3 value, is exactly q * 2^-9
// (subnormals below 8, the first binade above), so one v_cvt_pk_f32_fp8 converts two codes. The 2^9
// goes into the sub-block scale, which stays exact (a power of two).
__device__ __forceinline__ void fma_nib4(float &p, uint32_t nib4, float4 xv) {
    auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)nib4, false);  // bytes 0, 1
    auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)nib4, true);   // bytes 2, 3
    p = fmaf(lo[0], xv.x, p);
    p = fmaf(lo[1], xv.y, p);
    p = fmaf(hi[0], xv.z, p);
    p = fmaf(hi[1], xv.w, p);
}

// Eight lanes per row; lane (g, h) = (lane8 >> 1, lane8 & 1) owns the 16 qs bytes 32g + 16h .. +16 of
// every block: low nibbles are elements 16h..16h+15 of sub-block 2g, high nibbles the same elements of
// sub-block 2g+1. Each lane serves R rows (8 apart) with the same x, so a wave covers 8R rows and every x
// slice read from LDS feeds R rows. A workgroup is WAVES waves; with KS > 1 the waves form groups of KS on the
// same rows, each taking one KS-th of K (the parts meet in LDS and are added in part order), with KS = 1 each
// wave owns its rows' whole K. The 8 lanes of a row then add with a
// fixed xor-butterfly. x lives in LDS with a 16-byte pad per 256 bytes (the 8 slices a wave reads per step
// fall in distinct banks), its 16-element sums next to it. Weights are requested D blocks ahead, x one block
// ahead.
template <bool ACC, int D, int WAVES, int KS, int R>
__global__ __launch_bounds__(64 * WAVES) void gemv_fast_q4k(const Planes p, const float *__restrict__ x,
                                                            float *__restrict__ c, int64_t N, int64_t row0, int64_t K) {
    constexpr int THREADS = 64 * WAVES, ROWS = 8 * R * WAVES / KS;
    extern __shared__ float4 lds4[];
    __shared__ float part_lds[KS > 1 ? 64 * R * (WAVES / KS) * (KS - 1) : 1];
    const int nx4 = (int)(K / 4);
    float4 *xs = lds4;                                             // padded: nx4 + nx4/16 float4
    float *sx = reinterpret_cast<float *>(lds4 + nx4 + nx4 / 16);  // K/16 floats
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane8 = lane & 7, g = lane8 >> 1, hsel = lane8 & 1;
    const int rg = w / KS, part = w % KS;
    const int nb = (int)p.nb;
    const int nh = (nb + KS - 1) / KS;  // blocks per K part
    const int b0 = part * nh < nb ? part * nh : nb, b1 = b0 + nh < nb ? b0 + nh : nb;
    int64_t r[R];
    const uint4 *hp[R], *qp[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        r[i] = (int64_t)blockIdx.x * ROWS + 8 * R * rg + 8 * i + (lane >> 3);
        const int64_t row = row0 + (r[i] < N ? r[i] : N - 1);
        hp[i] = reinterpret_cast<const uint4 *>(p.aux) + row * nb;
        qp[i] = reinterpret_cast<const uint4 *>(p.qs) + row * nb * 8 + 4 * hsel + g;
    }
    uint4 H[D][R], Q[D][R];
#pragma unroll
    for (int s = 0; s < D; s++) {  // weights first: they come from HBM
        int b = b0 + s < b1 ? b0 + s : (b1 > b0 ? b1 - 1 : 0);
#pragma unroll
        for (int i = 0; i < R; i++) {
            H[s][i] = hp[i][b];
            Q[s][i] = qp[i][8 * b];
        }
    }
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int i = threadIdx.x; i < (int)(K / 16); i += THREADS) {
        float4 a = x4[4 * i], b = x4[4 * i + 1], cc = x4[4 * i + 2], dd = x4[4 * i + 3];
        float4 *o = xs + 4 * i + (i >> 2);  // padded index of 4i: 4i + (4i >> 4)
        o[0] = a;
        o[1] = b;
        o[2] = cc;
        o[3] = dd;
        sx[i] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) + ((cc.x + cc.y) + (cc.z + cc.w)) +
                ((dd.x + dd.y) + (dd.z + dd.w));
    }
    __syncthreads();
    const int k0 = (2 * g) & 3, k1 = (2 * g + 1) & 3;
    // x of elements 256b + 64g + 16h + 4c (+32 for the high nibbles): float4 64b + 16g + 4h + c, padded
    // by (64b + 16g + 4h + c) >> 4 = 4b + g
    const float4 *xg = xs + 17 * g + 4 * hsel;
    const float *sxg = sx + 4 * g + hsel;
    float4 XL[4], XH[4];
    {
        const float4 *xb = xg + 68 * (b0 < b1 ? b0 : 0);
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            XL[cc] = xb[cc];
            XH[cc] = xb[8 + cc];
        }
    }
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.0f;
    for (int bb = b0; bb < b1; bb += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            const int b = bb + s;
            uint4 h[R], q[R];
            const int nx = b + D < b1 ? b + D : b1 - 1;
#pragma unroll
            for (int i = 0; i < R; i++) {
                h[i] = H[s][i];
                q[i] = Q[s][i];
                H[s][i] = hp[i][nx];
                Q[s][i] = qp[i][8 * nx];
            }
            const float4 *xn = xg + 68 * (b + 1 < b1 ? b + 1 : b);
            float4 NL[4], NH[4];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                NL[cc] = xn[cc];
                NH[cc] = xn[8 + cc];
            }
            if (b < b1) {  // wave-uniform
                const float *sxb = sxg + 16 * b;
                const float sl = sxb[0], shx = sxb[2];
#pragma unroll
                for (int i = 0; i < R; i++) {
                    float d = f16_to_f32((uint16_t)(h[i].x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(h[i].x >> 16));
                    uint32_t sc_lo, sc_hi, m_lo, m_hi;
                    q4k_scales(h[i].y, h[i].z, h[i].w, sc_lo, sc_hi, m_lo, m_hi);
                    const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
                    const float d9 = d * 512.0f;  // undoes the 2^-9 of the fp8 reading
                    const float s0 = d9 * ubyte_f(scw, k0), n0 = -(dmin * ubyte_f(mw, k0));
                    const float s1 = d9 * ubyte_f(scw, k1), n1 = -(dmin * ubyte_f(mw, k1));
                    const uint32_t qw[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
                    float pl0 = 0.0f, pl1 = 0.0f, ph0 = 0.0f, ph1 = 0.0f;
#pragma unroll
                    for (int cc = 0; cc < 4; cc++) {
                        const uint32_t lo = qw[cc] & 0x0F0F0F0Fu, hi = (qw[cc] >> 4) & 0x0F0F0F0Fu;
                        float &pl = (cc & 1) ? pl1 : pl0;
                        float &ph = (cc & 1) ? ph1 : ph0;
                        fma_nib4(pl, lo, XL[cc]);
                        fma_nib4(ph, hi, XH[cc]);
                    }
                    acc[i] = fmaf(s0, pl0 + pl1, acc[i]);
                    acc[i] = fmaf(n0, sl, acc[i]);
                    acc[i] = fmaf(s1, ph0 + ph1, acc[i]);
                    acc[i] = fmaf(n1, shx, acc[i]);
                }
            }
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                XL[cc] = NL[cc];
                XH[cc] = NH[cc];
            }
        }
    }
    if (KS > 1) {  // parts 1..KS-1 hand their sums to part 0, which adds them in part order
        constexpr int RG = WAVES / KS;
        if (part) {
#pragma unroll
            for (int i = 0; i < R; i++) part_lds[64 * (((part - 1) * RG + rg) * R + i) + lane] = acc[i];
        }
        __syncthreads();
        if (part) return;
#pragma unroll
        for (int q = 1; q < KS; q++)
#pragma unroll
            for (int i = 0; i < R; i++) acc[i] = acc[i] + part_lds[64 * (((q - 1) * RG + rg) * R + i) + lane];
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
        float a = acc[i];
        a += __shfl_xor(a, 1);
        a += __shfl_xor(a, 2);
        a += __shfl_xor(a, 4);
        if (lane8 == 0 && r[i] < N) c[r[i]] = ACC ? c[r[i]] + a : a;
    }
}

template <int D, int WAVES, int KS, int R>
int run_q4k(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc) {
    constexpr int ROWS = 8 * R * WAVES / KS;
    const int64_t nx4 = w->K / 4;
    size_t lds = (size_t)(nx4 + nx4 / 16) * sizeof(float4) + (size_t)(w->K / 16) * sizeof(float);
    if (lds > 150 * 1024) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemv_fast: K too large for the LDS copy of x");
    dim3 grid((unsigned)((N + ROWS - 1) / ROWS)), block(64 * WAVES);
    if (acc)
        hipLaunchKernelGGL((gemv_fast_q4k<true, D, WAVES, KS, R>), grid, block, lds, ctx->stream, w->planes(), x, c, N, row0, w->K);
    else
        hipLaunchKernelGGL((gemv_fast_q4k<false, D, WAVES, KS, R>), grid, block, lds, ctx->stream, w->planes(), x, c, N, row0, w->K);
    return launch_check(ctx, "gemv_fast_q4k");
}

}  // namespace

int launch_gemv(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc,
                int mode);

int launch_gemv_fast(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     bool acc) {
    if (w->dtype == kQ4K) {
        // launch shape "D,WAVES,KS,R": blocks in flight per lane, waves per workgroup, K parts per row group,
        // rows per lane. Measured on cold 1.1 GiB rings: splitting K wins while the grid is small (1024 / 4096 rows
        // at K = 4096: 5.5 / 5.9 us with 2 parts vs 7.9 / 8.2 whole), whole rows per wave win from ~8192 rows
        // (14336 rows: 10.7-11.5 us vs 11.6-11.7). More blocks in flight or more rows per lane were slower.
        // TRHIP_FAST_CFG overrides.
        static const int forced = [] {
            const char *e = getenv("TRHIP_FAST_CFG");
            int d = 0, wv = 0, ks = 0, rr = 0;
            if (e && sscanf(e, "%d,%d,%d,%d", &d, &wv, &ks, &rr) == 4) return 1000 * d + 100 * wv + 10 * ks + rr;
            return 0;
        }();
        // K split in 4 for fewer rows (cold, us): 4096x14336 10.9 vs 14.5 (2 parts), 4096x4096 5.1 vs 6.0,
        // 1024x14336 8.3 vs 12.8
        const int cfg = forced ? forced : (N >= 8192 ? 2411 : (N >= 2048 ? 2841 : 2441));
        switch (cfg) {
        case 2441: return run_q4k<2, 4, 4, 1>(ctx, w, row0, N, x, c, acc);
        case 2841: return run_q4k<2, 8, 4, 1>(ctx, w, row0, N, x, c, acc);
        case 2421: return run_q4k<2, 4, 2, 1>(ctx, w, row0, N, x, c, acc);
        case 2411: return run_q4k<2, 4, 1, 1>(ctx, w, row0, N, x, c, acc);
        case 2422: return run_q4k<2, 4, 2, 2>(ctx, w, row0, N, x, c, acc);
        case 8421: return run_q4k<8, 4, 2, 1>(ctx, w, row0, N, x, c, acc);
        }
        return run_q4k<2, 4, 2, 1>(ctx, w, row0, N, x, c, acc);
    }
    return launch_gemv(ctx, w, row0, N, x, c, acc, TRHIP_MODE_EXACT);
}

}  // namespace trhip
