// actq.hip -- quantized-activation matmul (TR_quantized_activations): device quantizeQ8 and the
// integer block kernels, bit-identical to tensor/cpu_quant_q8.go.
//
// quantizeQ8 (cpu_quant_q8.go:39-68): per block of blk elements, amax = max|x|, id = fl(127/amax);
// if !(amax > 0) or id is not finite the block's codes and scale are 0, else d = fl(amax/127) and
// code = clamp(rne(fl(x*id)), +-127); bs = int16 sums of 16 codes. Division is IEEE (correctly
// rounded), rintf is round-to-nearest-even, nothing is fused (-ffp-contract=off).
//
// Block kernels: integer sums are exact in int32 by construction (the reference's own bound
// |isum| <= 8*63*32*15*127 < 2^31); the per-block float epilogue keeps the Go twins' rounding order:
//   q4  : t = fl(d_w*d8);                      acc = fl(acc + fl(t*fl(isum)))        (:74-87)
//   q4_k: t = fl(fl(d*fl(isum)) - fl(dmin*fl(msum))); acc = fl(acc + fl(t*d8))       (:91-116)
//   q6_k: t = fl(d*fl(isum - 32*msum));        acc = fl(acc + fl(t*d8))              (:378-407)
// blocks strictly in order. A row of x holding NaN/Inf takes the fp32 path (quantGemv) on its own
// (cpu_quant_q8.go:186-194): the quantizer flags it and the kernel computes that row's outputs with
// the exact fp32 dot (sdot32 order) instead. The quantizer writes one flag byte per activation block
// (plain stores, so no buffer has to be cleared first).
#include "trhip_internal.hpp"

namespace trhip {
namespace {

// TILED (blk 256, for the prefill MFMA kernels): codes, scales and (q4_k, sj not null) msum operands go to the tiled
// layout of prefill.hip (tiled_q / tiled_d / tiled_sj) instead of row-major, and no 16-sums are written.
template <int BLK, bool TILED = false>
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float *__restrict__ x, int64_t M, int64_t K,
                                                          int8_t *__restrict__ q, float *__restrict__ d,
                                                          int16_t *__restrict__ bs, uint8_t *__restrict__ bad_blk,
                                                          uint16_t *__restrict__ sj) {
    constexpr int TPB = BLK / 4;  // threads per activation block
    const int64_t nbk = K / BLK;
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = M * nbk * TPB;
    const bool live = gt < total;
    const int64_t gtc = live ? gt : total - 1;
    const int l4 = (int)(gtc % TPB);
    const int64_t blk_id = gtc / TPB;  // = m * nbk + b
    const int64_t off = blk_id * BLK + 4 * l4;  // element offset in x (rows are contiguous: m*K + b*BLK)
    float4 v = *reinterpret_cast<const float4 *>(x + off);
    float a = 0.0f;
    float av[4] = {fabsf(v.x), fabsf(v.y), fabsf(v.z), fabsf(v.w)};
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (av[i] > a) a = av[i];
    int bad = ((v.x - v.x) != 0.0f) | ((v.y - v.y) != 0.0f) | ((v.z - v.z) != 0.0f) | ((v.w - v.w) != 0.0f);
#pragma unroll
    for (int s = 1; s < TPB; s <<= 1) {
        float o = __shfl_xor(a, s);
        if (o > a) a = o;
        bad |= __shfl_xor(bad, s);
    }
    if (!live) return;
    if (l4 == 0) bad_blk[blk_id] = (uint8_t)(bad != 0);
    float id = 127.0f / a;
    float dv;
    int c[4];
    if (!(a > 0.0f) || (id - id) != 0.0f) {
        dv = 0.0f;
        c[0] = c[1] = c[2] = c[3] = 0;
    } else {
        dv = a / 127.0f;
        float xv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float t = rintf(xv[i] * id);
            t = fminf(fmaxf(t, -127.0f), 127.0f);
            c[i] = (int)t;
        }
    }
    uint32_t packed = (uint32_t)(c[0] & 0xFF) | ((uint32_t)(c[1] & 0xFF) << 8) | ((uint32_t)(c[2] & 0xFF) << 16) |
                      ((uint32_t)(c[3] & 0xFF) << 24);
    const int64_t m = blk_id / nbk, b = blk_id % nbk;
    if (TILED) {
        *reinterpret_cast<uint32_t *>(q + tiled_q(m, b, nbk, 4 * l4)) = packed;
        if (l4 == 0) d[tiled_d(m, b, nbk)] = dv;
    } else {
        *reinterpret_cast<uint32_t *>(q + off) = packed;
        if (l4 == 0) d[blk_id] = dv;
    }
    int s16 = c[0] + c[1] + c[2] + c[3];
    s16 += __shfl_xor(s16, 1);
    s16 += __shfl_xor(s16, 2);
    if (!TILED && (l4 & 3) == 0) bs[off / 16] = (int16_t)s16;
    if (TILED && sj) {  // q4_k: msum operands
        const int s32 = s16 + __shfl_xor(s16, 4);
        if ((l4 & 7) == 0) {
            const int j = l4 >> 3, sh = s32 >> 6, sl = s32 & 63;
            sj[tiled_sj(m, b, nbk, 0, j)] = __builtin_bit_cast(uint16_t, (_Float16)(float)sh);
            sj[tiled_sj(m, b, nbk, 1, j)] = __builtin_bit_cast(uint16_t, (_Float16)(float)sl);
        }
    } else if (BLK == 256 && sj) {
        // 32-element sums S_j = 64*Sh + Sl (Sh = floor(S/64) in [-64, 63], Sl in [0, 63]) as f16 operands of the
        // q4_k prefill kernel's msum product: [Sh_0..Sh_7, Sl_0..Sl_7] per activation block.
        const int s32 = s16 + __shfl_xor(s16, 4);
        if ((l4 & 7) == 0) {
            const int j = l4 >> 3, sh = s32 >> 6, sl = s32 & 63;
            sj[blk_id * 16 + j] = __builtin_bit_cast(uint16_t, (_Float16)(float)sh);
            sj[blk_id * 16 + 8 + j] = __builtin_bit_cast(uint16_t, (_Float16)(float)sl);
        }
    }
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// One thread per output (m, n); blocks in order. Correct for every M; the int8-MFMA kernel
// (actq_mfma.hip) takes the large-M shapes.
template <int DT, bool ACC>
__global__ __launch_bounds__(256) void actq_valu_kernel(const Planes p, int64_t N, int64_t row0, int64_t K,
                                                        const float *__restrict__ x, const int8_t *__restrict__ q,
                                                        const float *__restrict__ d8, const int16_t *__restrict__ bs,
                                                        const uint8_t *__restrict__ bad_blk, float *__restrict__ c) {
    const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t m = blockIdx.y;
    if (n >= N) return;
    const int64_t row = row0 + n;
    const int64_t nb = p.nb;
    float acc = 0.0f;
    bool row_bad = false;
    for (int64_t b = 0; b < nb; b++) row_bad |= bad_blk[m * nb + b] != 0;
    if (row_bad) {
        acc = exact_dot_row<DT>(p, row, x + m * K, K);
    } else if (DT == kQ4) {
        const uint32_t *qa = reinterpret_cast<const uint32_t *>(q + m * K);
        const int16_t *bm = bs + m * (K / 16);
        const float *dm = d8 + m * nb;
        for (int64_t b = 0; b < nb; b++) {
            int64_t bi = row * nb + b;
            uint4 w = *reinterpret_cast<const uint4 *>(p.qs + bi * 16);
            uint32_t wd[4] = {w.x, w.y, w.z, w.w};
            int s = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                s = sdot4(wd[i] & 0x0F0F0F0Fu, qa[8 * b + i], s);
                s = sdot4((wd[i] >> 4) & 0x0F0F0F0Fu, qa[8 * b + 4 + i], s);
            }
            int isum = s - 8 * ((int)bm[2 * b] + (int)bm[2 * b + 1]);
            float t = f16_to_f32(p.d[bi]) * dm[b];
            acc = acc + t * (float)isum;
        }
    } else if (DT == kQ4K) {
        const uint32_t *qa = reinterpret_cast<const uint32_t *>(q + m * K);
        const int16_t *bm = bs + m * (K / 16);
        const float *dm = d8 + m * nb;
        for (int64_t b = 0; b < nb; b++) {
            int64_t bi = row * nb + b;
            uint4 h = *reinterpret_cast<const uint4 *>(p.aux + bi * 16);
            const uint32_t *qw = reinterpret_cast<const uint32_t *>(p.qs + bi * 128);
            uint32_t sc_lo, sc_hi, m_lo, m_hi;
            q4k_scales(h.y, h.z, h.w, sc_lo, sc_hi, m_lo, m_hi);
            int isum = 0, msum = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                int g = j >> 1;
                int s = 0;
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        uint32_t wv = qw[q4k_pos(32 * g + 8 * t + 4 * hh) / 4];
                        uint32_t nib = (j & 1) ? ((wv >> 4) & 0x0F0F0F0Fu) : (wv & 0x0F0F0F0Fu);
                        s = sdot4(nib, qa[64 * b + 8 * j + 2 * t + hh], s);
                    }
                uint32_t scw = j < 4 ? sc_lo : sc_hi, mw = j < 4 ? m_lo : m_hi;
                int scj = (int)((scw >> (8 * (j & 3))) & 0xFF), mj = (int)((mw >> (8 * (j & 3))) & 0xFF);
                isum += scj * s;
                msum += mj * ((int)bm[16 * b + 2 * j] + (int)bm[16 * b + 2 * j + 1]);
            }
            float dd = f16_to_f32((uint16_t)(h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(h.x >> 16));
            float t = (dd * (float)isum) - (dmin * (float)msum);
            acc = acc + t * dm[b];
        }
    } else if (DT == kQ6K) {
        const uint32_t *qa = reinterpret_cast<const uint32_t *>(q + m * K);
        const int16_t *bm = bs + m * (K / 16);
        const float *dm = d8 + m * nb;
        for (int64_t b = 0; b < nb; b++) {
            int64_t bi = row * nb + b;
            const uint32_t *lw = reinterpret_cast<const uint32_t *>(p.qs + bi * 128);
            const uint32_t *hw = reinterpret_cast<const uint32_t *>(p.aux + bi * 64);
            const int8_t *sc = reinterpret_cast<const int8_t *>(p.sc + bi * 16);
            int isum = 0, msum = 0;
#pragma unroll
            for (int n2 = 0; n2 < 2; n2++)
#pragma unroll
                for (int k = 0; k < 4; k++)
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        int s = 0;
#pragma unroll
                        for (int hh = 0; hh < 2; hh++) {
                            uint32_t A = lw[8 * t + 4 * n2 + hh], B = lw[8 * t + 4 * n2 + 2 + hh];
                            uint32_t H = hw[4 * t + 2 * n2 + hh];
                            uint32_t cw;
                            if (k == 0) cw = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
                            else if (k == 1) cw = (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
                            else if (k == 2) cw = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
                            else cw = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
                            s = sdot4(cw, qa[64 * b + 32 * n2 + 8 * k + 2 * t + hh], s);
                        }
                        isum += (int)sc[8 * n2 + 2 * k + (t >> 1)] * s;
                    }
#pragma unroll
            for (int j = 0; j < 16; j++) msum += (int)sc[j] * (int)bm[16 * b + j];
            float t = f16_to_f32(p.d[bi]) * (float)(isum - 32 * msum);
            acc = acc + t * dm[b];
        }
    }
    float *o = c + m * N + n;
    if (ACC) *o = *o + acc;
    else *o = acc;
}

template <int DT>
int run_valu(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, int64_t M,
             bool acc, const int8_t *q, const float *d, const int16_t *bs, const uint8_t *bad) {
    dim3 grid((unsigned)((N + 255) / 256), (unsigned)M), block(256);
    if (acc)
        hipLaunchKernelGGL((actq_valu_kernel<DT, true>), grid, block, 0, ctx->stream, w->planes(), N, row0, w->K, x, q, d, bs, bad, c);
    else
        hipLaunchKernelGGL((actq_valu_kernel<DT, false>), grid, block, 0, ctx->stream, w->planes(), N, row0, w->K, x, q, d, bs, bad, c);
    return launch_check(ctx, "actq_valu");
}

}  // namespace

int launch_quantize_tiles(trhip_ctx *ctx, const float *x, int64_t M, int64_t K, int8_t *qt, float *dt, uint16_t *st,
                          uint8_t *bad) {
    if (M == 0 || K == 0) return TRHIP_OK;
    const int64_t total = M * K / 4;
    hipLaunchKernelGGL((quantize_q8_kernel<256, true>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream,
                       x, M, K, qt, dt, nullptr, bad, st);
    return launch_check(ctx, "quantize_tiles");
}

int launch_quantize_q8(trhip_ctx *ctx, const float *x, int64_t M, int64_t K, int blk, int8_t *q, float *d, int16_t *bs,
                       uint8_t *bad, uint16_t *sj) {
    if (M == 0 || K == 0) return TRHIP_OK;
    int64_t total = M * K / 4;
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    if (blk == 256)
        hipLaunchKernelGGL(quantize_q8_kernel<256>, grid, block, 0, ctx->stream, x, M, K, q, d, bs, bad, sj);
    else
        hipLaunchKernelGGL(quantize_q8_kernel<32>, grid, block, 0, ctx->stream, x, M, K, q, d, bs, bad, nullptr);
    return launch_check(ctx, "quantize_q8");
}

// Below this many activation rows the thread-per-output kernel wins (the MFMA tile is 128 rows).
constexpr int64_t kActqMfmaMinRows = 8;

int launch_actq_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     int64_t M, bool acc, const int8_t *q, const float *d, const uint16_t *sj, const uint8_t *bad,
                     bool fast);

// fast: the matrix-core kernel's fused epilogue (tolerance); the thread-per-output kernel is exact either way.
int launch_actq(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, int64_t M,
                bool acc, const int8_t *q, const float *d, const int16_t *bs, const uint8_t *bad, const uint16_t *sj,
                bool fast) {
    if (N == 0 || M == 0) return TRHIP_OK;
    switch (w->dtype) {
    case kQ4:
        if (actq4_mfma_applies(M, N, row0, w->K)) return launch_actq4_mfma(ctx, w, row0, N, x, c, M, acc, q, d, bad);
        return run_valu<kQ4>(ctx, w, row0, N, x, c, M, acc, q, d, bs, bad);
    case kQ4K:
        if (M >= kActqMfmaMinRows && sj) return launch_actq_mfma(ctx, w, row0, N, x, c, M, acc, q, d, sj, bad, fast);
        return run_valu<kQ4K>(ctx, w, row0, N, x, c, M, acc, q, d, bs, bad);
    case kQ6K:
        if (actq6_mfma_applies(M, N, row0, w->K)) return launch_actq6_mfma(ctx, w, row0, N, x, c, M, acc, q, d, bad);
        return run_valu<kQ6K>(ctx, w, row0, N, x, c, M, acc, q, d, bs, bad);
    }
    return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq: dtype must be q4, q4_k or q6_k");
}

}  // namespace trhip
