// gemv.hip -- decode GEMV (M == 1) with fp32 activations, bit-identical to TR's CPU quantDot.
//
// The reference's result is dequant + sdot32 (tensor/cpu_quant_amd64.s:3-6, cpu_gemv_amd64.s:190-227):
// element i of a row is fused (fmaf) into chain i mod 32 in ascending i; the chains are then summed as
// Y[l] = (A0[l]+A1[l]) + (A2[l]+A3[l]) with A_a[l] = chain 8a+l, s_l = Y[l]+Y[l+4], r = (s0+s2)+(s1+s3).
//
// Mapping: one row per quad of lanes; lane t (0..3) owns the eight chains 8t..8t+7 (the sdot32 register
// A_t), i.e. elements 32G + 8t + l of every 32-element group G, processed in ascending G. The first two
// levels of the tree are exchanged inside the quad with xor-shuffles (IEEE addition is commutative, so
// both partners hold the same bits), the rest is in-lane. Dequantized values are produced exactly as in
// tensor/quant.go: exact products, one rounding where the reference rounds (fmaf of exact operands).
//
// Bandwidth: every weight byte is read once, with 128-bit loads where the plane layout allows; x is
// read through the cache (it is shared by all rows).
#include "trhip_internal.hpp"

namespace trhip {
namespace {

constexpr int kRowsPerWG = 16;  // 64 threads: 16 rows x 4 lanes

__device__ __forceinline__ void fma4(float *acc, uint32_t codes, float s, float negm, float4 xv) {
    acc[0] = fmaf(fmaf(s, ubyte_f(codes, 0), negm), xv.x, acc[0]);
    acc[1] = fmaf(fmaf(s, ubyte_f(codes, 1), negm), xv.y, acc[1]);
    acc[2] = fmaf(fmaf(s, ubyte_f(codes, 2), negm), xv.z, acc[2]);
    acc[3] = fmaf(fmaf(s, ubyte_f(codes, 3), negm), xv.w, acc[3]);
}

// One 32-element group for this lane: 8 codes (two dwords), value = fmaf(s, code, negm).
__device__ __forceinline__ void group8(float *acc, uint32_t c0, uint32_t c1, float s, float negm,
                                       const float4 *__restrict__ xg) {
    float4 xa = xg[0], xb = xg[1];
    fma4(acc, c0, s, negm, xa);
    fma4(acc + 4, c1, s, negm, xb);
}

__device__ __forceinline__ float sdot32_tree(float *acc) {
    float Y[8];
#pragma unroll
    for (int l = 0; l < 8; l++) {
        float p = acc[l] + __shfl_xor(acc[l], 1);
        Y[l] = p + __shfl_xor(p, 2);
    }
    float s0 = Y[0] + Y[4], s1 = Y[1] + Y[5], s2 = Y[2] + Y[6], s3 = Y[3] + Y[7];
    return (s0 + s2) + (s1 + s3);
}

template <int DT, bool ACC>
__global__ __launch_bounds__(64) void gemv_exact_kernel(const Planes p, const float *__restrict__ x,
                                                        float *__restrict__ c, int64_t N, int64_t row0) {
    const int t = threadIdx.x & 3;
    const int64_t r = (int64_t)blockIdx.x * kRowsPerWG + (threadIdx.x >> 2);
    if (r >= N) return;  // the whole quad leaves together
    const int64_t row = row0 + r;
    const int64_t nb = p.nb;
    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; l++) acc[l] = 0.0f;
    // element 32G + 8t -> float4 index 8G + 2t
    const float4 *__restrict__ xv = reinterpret_cast<const float4 *>(x) + 2 * t;

    if (DT == kQ8) {
        const uint2 *__restrict__ qp = reinterpret_cast<const uint2 *>(p.qs + row * nb * 32) + t;
        const uint16_t *__restrict__ dp = p.d + row * nb;
        for (int64_t b = 0; b < nb; b++) {
            uint2 q = qp[4 * b];
            float d = f16_to_f32(dp[b]);
            // code = u - 128 with u = byte ^ 0x80; value (u-128)*d is exact, so fmaf(d, u, -128d) is too
            group8(acc, q.x ^ 0x80808080u, q.y ^ 0x80808080u, d, -128.0f * d, xv + 8 * b);
        }
    } else if (DT == kQ4) {
        const uint2 *__restrict__ qp = reinterpret_cast<const uint2 *>(p.qs + row * nb * 16) + (t & 1);
        const uint16_t *__restrict__ dp = p.d + row * nb;
        const int sh = (t & 2) ? 4 : 0;  // lanes 2,3 take the high nibbles (elements 16..31)
        for (int64_t b = 0; b < nb; b++) {
            uint2 q = qp[2 * b];
            float d = f16_to_f32(dp[b]);
            group8(acc, (q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu, d, -8.0f * d, xv + 8 * b);
        }
    } else if (DT == kQ4K) {
        const uint4 *__restrict__ hp = reinterpret_cast<const uint4 *>(p.aux + row * nb * 16);
        const uint4 *__restrict__ qp = reinterpret_cast<const uint4 *>(p.qs + row * nb * 128 + 32 * t);
        for (int64_t b = 0; b < nb; b++) {
            uint4 h = hp[b];
            uint4 qa = qp[8 * b], qb = qp[8 * b + 1];
            float d = f16_to_f32((uint16_t)(h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(h.x >> 16));
            float d16 = d * 0.0625f;
            uint32_t sc_lo, sc_hi, m_lo, m_hi;
            q4k_scales(h.y, h.z, h.w, sc_lo, sc_hi, m_lo, m_hi);
            const float4 *xb = xv + 64 * b;
            uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
            for (int g = 0; g < 4; g++) {
                uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
                int k0 = (2 * g) & 3, k1 = (2 * g + 1) & 3;
                float s0 = d * ubyte_f(scw, k0), n0 = -(dmin * ubyte_f(mw, k0));
                float s1 = d16 * ubyte_f(scw, k1), n1 = -(dmin * ubyte_f(mw, k1));
                // sub-block 2g: low nibbles; sub-block 2g+1: high nibbles used as 16*code (scale d/16)
                group8(acc, w[2 * g] & 0x0F0F0F0Fu, w[2 * g + 1] & 0x0F0F0F0Fu, s0, n0, xb + 8 * (2 * g));
                group8(acc, w[2 * g] & 0xF0F0F0F0u, w[2 * g + 1] & 0xF0F0F0F0u, s1, n1, xb + 8 * (2 * g + 1));
            }
        }
    } else {  // q6_k
        const uint4 *__restrict__ lp = reinterpret_cast<const uint4 *>(p.qs + row * nb * 128 + 32 * t);
        const uint4 *__restrict__ hp = reinterpret_cast<const uint4 *>(p.aux + row * nb * 64 + 16 * t);
        const uint4 *__restrict__ sp = reinterpret_cast<const uint4 *>(p.sc + row * nb * 16);
        const uint16_t *__restrict__ dp = p.d + row * nb;
        const int th = t >> 1;
        for (int64_t b = 0; b < nb; b++) {
            uint4 la = lp[8 * b], lb = lp[8 * b + 1], hh = hp[4 * b], sv = sp[b];
            float d = f16_to_f32(dp[b]);
            uint32_t scw[4] = {sv.x, sv.y, sv.z, sv.w};
            const float4 *xb = xv + 64 * b;
#pragma unroll
            for (int n = 0; n < 2; n++) {
                uint32_t A0 = n ? lb.x : la.x, A1 = n ? lb.y : la.y;  // ql[64n + 8t + l]
                uint32_t B0 = n ? lb.z : la.z, B1 = n ? lb.w : la.w;  // ql[64n + 32 + 8t + l]
                uint32_t H0 = n ? hh.z : hh.x, H1 = n ? hh.w : hh.y;  // qh[32n + 8t + l]
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    uint32_t c0, c1;
                    if (k == 0) {
                        c0 = (A0 & 0x0F0F0F0Fu) | ((H0 << 4) & 0x30303030u);
                        c1 = (A1 & 0x0F0F0F0Fu) | ((H1 << 4) & 0x30303030u);
                    } else if (k == 1) {
                        c0 = (B0 & 0x0F0F0F0Fu) | ((H0 << 2) & 0x30303030u);
                        c1 = (B1 & 0x0F0F0F0Fu) | ((H1 << 2) & 0x30303030u);
                    } else if (k == 2) {
                        c0 = ((A0 >> 4) & 0x0F0F0F0Fu) | (H0 & 0x30303030u);
                        c1 = ((A1 >> 4) & 0x0F0F0F0Fu) | (H1 & 0x30303030u);
                    } else {
                        c0 = ((B0 >> 4) & 0x0F0F0F0Fu) | ((H0 >> 2) & 0x30303030u);
                        c1 = ((B1 >> 4) & 0x0F0F0F0Fu) | ((H1 >> 2) & 0x30303030u);
                    }
                    int si = 8 * n + 2 * k + th;  // 16-element sub-block of these 8 elements
                    int8_t scv = (int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xFF);
                    float ds = d * (float)scv;  // exact (11 x 8 bits)
                    // value fl(ds*(code-32)) == fmaf(ds, code, -32*ds): same real number, one rounding
                    group8(acc, c0, c1, ds, -32.0f * ds, xb + 8 * (4 * n + k));
                }
            }
        }
    }
    float res = sdot32_tree(acc);
    if (t == 0) {
        if (ACC) c[r] = c[r] + res;
        else c[r] = res;
    }
}

template <int DT>
int launch_exact(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                 bool acc) {
    dim3 grid((unsigned)((N + kRowsPerWG - 1) / kRowsPerWG)), block(64);
    if (acc)
        hipLaunchKernelGGL((gemv_exact_kernel<DT, true>), grid, block, 0, ctx->stream, w->planes(), x, c, N, row0);
    else
        hipLaunchKernelGGL((gemv_exact_kernel<DT, false>), grid, block, 0, ctx->stream, w->planes(), x, c, N, row0);
    return launch_check(ctx, "gemv_exact");
}

}  // namespace

int launch_gemv_fast(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     bool acc);

int launch_gemv(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc,
                int mode) {
    if (N == 0) return TRHIP_OK;
    if (mode == TRHIP_MODE_FAST) return launch_gemv_fast(ctx, w, row0, N, x, c, acc);
    switch (w->dtype) {
    case kQ8: return launch_exact<kQ8>(ctx, w, row0, N, x, c, acc);
    case kQ4: return launch_exact<kQ4>(ctx, w, row0, N, x, c, acc);
    case kQ4K: return launch_exact<kQ4K>(ctx, w, row0, N, x, c, acc);
    case kQ6K: return launch_exact<kQ6K>(ctx, w, row0, N, x, c, acc);
    }
    return fail(ctx, TRHIP_ERR_INVALID, "gemv: bad dtype");
}

}  // namespace trhip
