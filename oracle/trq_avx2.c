/*
 * trq_avx2.c -- AVX2/FMA/F16C restatement of the reference's quant-dot assembly: the timed
 * CPU baseline ("port") and a second, independent restatement that the scalar oracle must
 * agree with bit for bit (test infrastructure only; the product never calls it).
 *
 * fp32-activation kernels follow internal/compute/tensor/cpu_quant_amd64.s and
 * cpu_gemv_amd64.s instruction by instruction (same accumulator/lane assignment, same
 * FMA/FMSUB placement, same final SUM32 tree). The integer act-quant kernels compute the
 * same exact integer block sums as cpu_quant_q8.go's Go twins (the reference's own
 * sdotq4kq8/sdotq6kq8/sdotq4q8 are bit-identical to those twins, cpu_quant_q8_test.go:54-91)
 * and then apply the twins' explicitly rounded per-block float epilogue in block order.
 */
#include "trq_oracle.h"

#include <immintrin.h>
#include <stdlib.h>
#include <string.h>

int trq_avx2_available(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

/* SUM32 macro, cpu_quant_amd64.s:9-18 */
static inline float sum32(__m256 y0, __m256 y1, __m256 y2, __m256 y3) {
    y0 = _mm256_add_ps(y0, y1);
    y2 = _mm256_add_ps(y2, y3);
    y0 = _mm256_add_ps(y0, y2);
    __m128 x0 = _mm256_castps256_ps128(y0);
    __m128 x1 = _mm256_extractf128_ps(y0, 1);
    x0 = _mm_add_ps(x0, x1);
    x1 = _mm_movehl_ps(x1, x0);
    x0 = _mm_add_ps(x0, x1);
    x1 = _mm_movehdup_ps(x0);
    x0 = _mm_add_ss(x0, x1);
    return _mm_cvtss_f32(x0);
}

static inline __m256 bcast_f16(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    __m128 v = _mm_cvtph_ps(_mm_cvtsi32_si128(h));
    return _mm256_broadcastss_ps(v);
}

/* cpu_gemv_amd64.s:190-227 */
__attribute__((target("avx2,fma,f16c")))
float trq_avx2_sdot32(size_t n, const float *x, const float *y) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (size_t i = 0; i + 32 <= n; i += 32) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), _mm256_loadu_ps(y + i), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 8), _mm256_loadu_ps(y + i + 8), a1);
        a2 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 16), _mm256_loadu_ps(y + i + 16), a2);
        a3 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 24), _mm256_loadu_ps(y + i + 24), a3);
    }
    return sum32(a0, a1, a2, a3);
}

/* sdotq8, cpu_quant_amd64.s:83-109 (Q8LANE :27-31) */
__attribute__((target("avx2,fma,f16c")))
static float sdotq8(size_t n, const float *x, const uint8_t *w) {
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (size_t b = 0; b < n / 32; b++, w += 34, x += 32) {
        __m256 d = bcast_f16(w);
        for (int k = 0; k < 4; k++) {
            __m128i c8 = _mm_loadl_epi64((const __m128i *)(w + 2 + 8 * k));
            __m256 v = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(c8)), d);
            acc[k] = _mm256_fmadd_ps(v, _mm256_loadu_ps(x + 8 * k), acc[k]);
        }
    }
    return sum32(acc[0], acc[1], acc[2], acc[3]);
}

/* sdotq4, cpu_quant_amd64.s:130-160 (Q40LANE :113-124) */
__attribute__((target("avx2,fma,f16c")))
static float sdotq4(size_t n, const float *x, const uint8_t *w) {
    __m256 y0 = _mm256_setzero_ps(), y1 = y0, y2 = y0, y3 = y0;
    const __m256i f15 = _mm256_set1_epi32(15), e8 = _mm256_set1_epi32(8);
    for (size_t b = 0; b < n / 32; b++, w += 18, x += 32) {
        __m256 d = bcast_f16(w);
        for (int k = 0; k < 2; k++) {
            __m128i c8 = _mm_loadl_epi64((const __m128i *)(w + 2 + 8 * k));
            __m256i v = _mm256_cvtepu8_epi32(c8);
            __m256i lo = _mm256_sub_epi32(_mm256_and_si256(f15, v), e8);
            __m256i hi = _mm256_sub_epi32(_mm256_srli_epi32(v, 4), e8);
            __m256 fl = _mm256_mul_ps(_mm256_cvtepi32_ps(lo), d);
            __m256 fh = _mm256_mul_ps(_mm256_cvtepi32_ps(hi), d);
            if (k == 0) {
                y0 = _mm256_fmadd_ps(fl, _mm256_loadu_ps(x + 0), y0);
                y2 = _mm256_fmadd_ps(fh, _mm256_loadu_ps(x + 16), y2);
            } else {
                y1 = _mm256_fmadd_ps(fl, _mm256_loadu_ps(x + 8), y1);
                y3 = _mm256_fmadd_ps(fh, _mm256_loadu_ps(x + 24), y3);
            }
        }
    }
    return sum32(y0, y1, y2, y3);
}

/* sdotq4k, cpu_quant_amd64.s:179-268 (Q4LANE :165-174). The scale scratch holds per group
 * [d*a_lo, m*b_lo, (d/16)*a_hi, m*b_hi]; the high nibble is used unshifted (16*code). */
__attribute__((target("avx2,fma,f16c")))
static float sdotq4k(size_t blocks, const float *x, const uint8_t *w) {
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    const __m256i f15 = _mm256_set1_epi32(15), f0 = _mm256_set1_epi32(0xF0);
    float sc[16];
    for (size_t b = 0; b < blocks; b++) {
        float d = trq_f16_to_f32((uint16_t)(w[0] | (w[1] << 8)));
        float dmin = trq_f16_to_f32((uint16_t)(w[2] | (w[3] << 8)));
        /* VMULPS Y6, Y7: d x [1, 1/16] alternating; then a/b bytes (0..63) times [d, d/16] and dmin. */
        for (int g = 0; g < 4; g++) {
            uint8_t a0, m0, a1, m1;
            trq_q4k_scale(2 * g, w + 4, &a0, &m0);
            trq_q4k_scale(2 * g + 1, w + 4, &a1, &m1);
            sc[4 * g + 0] = d * (float)a0;
            sc[4 * g + 1] = dmin * (float)m0;
            sc[4 * g + 2] = (d * 0.0625f) * (float)a1;
            sc[4 * g + 3] = dmin * (float)m1;
        }
        const uint8_t *q = w + 16;
        for (int g = 0; g < 4; g++, q += 32, x += 64) {
            __m256 y10 = _mm256_set1_ps(sc[4 * g + 0]), y11 = _mm256_set1_ps(sc[4 * g + 1]);
            __m256 y12 = _mm256_set1_ps(sc[4 * g + 2]), y13 = _mm256_set1_ps(sc[4 * g + 3]);
            for (int k = 0; k < 4; k++) {
                __m256i v = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)(q + 8 * k)));
                __m256 lo = _mm256_cvtepi32_ps(_mm256_and_si256(f15, v));
                __m256 hi = _mm256_cvtepi32_ps(_mm256_and_si256(f0, v));
                lo = _mm256_fmsub_ps(y10, lo, y11);
                hi = _mm256_fmsub_ps(y12, hi, y13);
                acc[k] = _mm256_fmadd_ps(lo, _mm256_loadu_ps(x + 8 * k), acc[k]);
                acc[k] = _mm256_fmadd_ps(hi, _mm256_loadu_ps(x + 32 + 8 * k), acc[k]);
            }
        }
        w += 144;
    }
    return sum32(acc[0], acc[1], acc[2], acc[3]);
}

/* sdotq6k, cpu_quant_amd64.s:273-327 (Q6CODES :50-78, Q6LANE :42-46). */
__attribute__((target("avx2,fma,f16c")))
static float sdotq6k(size_t blocks, const float *x, const uint8_t *w) {
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    const __m256i m0f = _mm256_set1_epi8(0x0F), m30 = _mm256_set1_epi8(0x30), c32 = _mm256_set1_epi8(32);
    float ds[16];
    int8_t codes[128];
    for (size_t b = 0; b < blocks; b++) {
        float d = trq_f16_to_f32((uint16_t)(w[208] | (w[209] << 8)));
        for (int j = 0; j < 16; j++) ds[j] = d * (float)(int8_t)w[192 + j];
        const uint8_t *ql = w, *qh = w + 128;
        for (int half = 0; half < 2; half++) {
            __m256i y8 = _mm256_loadu_si256((const __m256i *)ql);
            __m256i y9 = _mm256_loadu_si256((const __m256i *)(ql + 32));
            __m256i y10 = _mm256_loadu_si256((const __m256i *)qh);
            __m256i c0 = _mm256_sub_epi8(_mm256_or_si256(_mm256_and_si256(m0f, y8), _mm256_and_si256(m30, _mm256_slli_epi16(y10, 4))), c32);
            __m256i c1 = _mm256_sub_epi8(_mm256_or_si256(_mm256_and_si256(m0f, y9), _mm256_and_si256(m30, _mm256_slli_epi16(y10, 2))), c32);
            __m256i c2 = _mm256_sub_epi8(_mm256_or_si256(_mm256_and_si256(m0f, _mm256_srli_epi16(y8, 4)), _mm256_and_si256(m30, y10)), c32);
            __m256i c3 = _mm256_sub_epi8(_mm256_or_si256(_mm256_and_si256(m0f, _mm256_srli_epi16(y9, 4)), _mm256_and_si256(m30, _mm256_srli_epi16(y10, 2))), c32);
            _mm256_storeu_si256((__m256i *)(codes + 0), c0);
            _mm256_storeu_si256((__m256i *)(codes + 32), c1);
            _mm256_storeu_si256((__m256i *)(codes + 64), c2);
            _mm256_storeu_si256((__m256i *)(codes + 96), c3);
            /* Q6LANE(off=8k, s0, x0..x3, acc k): four steps, 32 codes apart, scales 8 apart. */
            for (int k = 0; k < 4; k++) {
                int s0 = (k < 2) ? 0 : 4;
                for (int st = 0; st < 4; st++) {
                    __m256 v = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)(codes + 8 * k + 32 * st))));
                    v = _mm256_mul_ps(_mm256_set1_ps(ds[half * 8 + (s0 + 8 * st) / 4]), v);
                    acc[k] = _mm256_fmadd_ps(v, _mm256_loadu_ps(x + 8 * k + 32 * st), acc[k]);
                }
            }
            ql += 64;
            qh += 32;
            x += 128; /* ADDQ $512, SI */
        }
        w += 210;
    }
    return sum32(acc[0], acc[1], acc[2], acc[3]);
}

float trq_avx2_quant_dot(int dt, const float *x, const uint8_t *w, size_t K) {
    switch (dt) {
    case TRQ_Q8: return sdotq8(K, x, w);
    case TRQ_Q4: return sdotq4(K, x, w);
    case TRQ_Q4K: return sdotq4k(K / 256, x, w);
    case TRQ_Q6K: return sdotq6k(K / 256, x, w);
    }
    return 0.0f;
}

void trq_avx2_quant_gemv(int dt, size_t N, size_t K, const float *x, const uint8_t *w, float *c,
                         int threads) {
    if (K == 0) return;
    size_t rb = K / (size_t)trq_block_elems(dt) * (size_t)trq_block_bytes(dt);
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(guided)
    for (long n = 0; n < (long)N; n++) c[n] = c[n] + trq_avx2_quant_dot(dt, x, w + (size_t)n * rb, K);
}

/* ---- act-quant integer block kernels (same exact integers as the Go twins) ---- */

__attribute__((target("avx2")))
static inline int32_t hsum_epi32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

/* sum of u8 (<=63) x s8 products over 32 lanes, exact */
__attribute__((target("avx2")))
static inline __m256i dot_u8s8(__m256i u, __m256i s) {
    return _mm256_madd_epi16(_mm256_maddubs_epi16(u, s), _mm256_set1_epi16(1));
}

__attribute__((target("avx2,fma,f16c")))
static float q4kq8_avx2(size_t blocks, const uint8_t *w, const int8_t *q, const float *d, const int16_t *bs) {
    float acc = 0.0f;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    for (size_t i = 0; i < blocks; i++, w += 144, q += 256, bs += 16) {
        float dd = trq_f16_to_f32((uint16_t)(w[0] | (w[1] << 8)));
        float dmin = trq_f16_to_f32((uint16_t)(w[2] | (w[3] << 8)));
        int32_t isum = 0, msum = 0;
        for (int g = 0; g < 4; g++) {
            __m256i qs = _mm256_loadu_si256((const __m256i *)(w + 16 + 32 * g));
            __m256i lo = _mm256_and_si256(qs, m4), hi = _mm256_and_si256(_mm256_srli_epi16(qs, 4), m4);
            int32_t s1 = hsum_epi32(dot_u8s8(lo, _mm256_loadu_si256((const __m256i *)(q + 64 * g))));
            int32_t s2 = hsum_epi32(dot_u8s8(hi, _mm256_loadu_si256((const __m256i *)(q + 64 * g + 32))));
            uint8_t sc1, m1, sc2, m2;
            trq_q4k_scale(2 * g, w + 4, &sc1, &m1);
            trq_q4k_scale(2 * g + 1, w + 4, &sc2, &m2);
            isum += (int32_t)sc1 * s1 + (int32_t)sc2 * s2;
            msum += (int32_t)m1 * (bs[4 * g] + bs[4 * g + 1]) + (int32_t)m2 * (bs[4 * g + 2] + bs[4 * g + 3]);
        }
        float t = (dd * (float)isum) - (dmin * (float)msum);
        acc = acc + t * d[i];
    }
    return acc;
}

__attribute__((target("avx2,fma,f16c")))
static float q6kq8_avx2(size_t blocks, const uint8_t *w, const int8_t *q, const float *d, const int16_t *bs) {
    float acc = 0.0f;
    const __m256i m0f = _mm256_set1_epi8(0x0F), m30 = _mm256_set1_epi8(0x30);
    for (size_t i = 0; i < blocks; i++, w += 210, q += 256, bs += 16) {
        float dd = trq_f16_to_f32((uint16_t)(w[208] | (w[209] << 8)));
        const int8_t *sc = (const int8_t *)(w + 192);
        int32_t isum = 0, msum = 0;
        for (int half = 0; half < 2; half++) {
            const uint8_t *ql = w + 64 * half, *qh = w + 128 + 32 * half;
            __m256i y8 = _mm256_loadu_si256((const __m256i *)ql);
            __m256i y9 = _mm256_loadu_si256((const __m256i *)(ql + 32));
            __m256i y10 = _mm256_loadu_si256((const __m256i *)qh);
            __m256i c[4];
            c[0] = _mm256_or_si256(_mm256_and_si256(m0f, y8), _mm256_and_si256(m30, _mm256_slli_epi16(y10, 4)));
            c[1] = _mm256_or_si256(_mm256_and_si256(m0f, y9), _mm256_and_si256(m30, _mm256_slli_epi16(y10, 2)));
            c[2] = _mm256_or_si256(_mm256_and_si256(m0f, _mm256_srli_epi16(y8, 4)), _mm256_and_si256(m30, y10));
            c[3] = _mm256_or_si256(_mm256_and_si256(m0f, _mm256_srli_epi16(y9, 4)), _mm256_and_si256(m30, _mm256_srli_epi16(y10, 2)));
            for (int k = 0; k < 4; k++) {
                /* codes c[k] cover elements 128*half + 32*k + (0..31): sub-blocks 2k, 2k+1 of the half */
                __m256i p = _mm256_maddubs_epi16(c[k], _mm256_loadu_si256((const __m256i *)(q + 128 * half + 32 * k)));
                __m256i s32 = _mm256_madd_epi16(p, _mm256_set1_epi16(1));
                __m128i lo = _mm256_castsi256_si128(s32), hi = _mm256_extracti128_si256(s32, 1);
                lo = _mm_add_epi32(lo, _mm_shuffle_epi32(lo, 0x4E));
                lo = _mm_add_epi32(lo, _mm_shuffle_epi32(lo, 0xB1));
                hi = _mm_add_epi32(hi, _mm_shuffle_epi32(hi, 0x4E));
                hi = _mm_add_epi32(hi, _mm_shuffle_epi32(hi, 0xB1));
                isum += (int32_t)sc[8 * half + 2 * k] * _mm_cvtsi128_si32(lo) +
                        (int32_t)sc[8 * half + 2 * k + 1] * _mm_cvtsi128_si32(hi);
            }
        }
        for (int j = 0; j < 16; j++) msum += (int32_t)sc[j] * (int32_t)bs[j];
        float t = dd * (float)(isum - 32 * msum);
        acc = acc + t * d[i];
    }
    return acc;
}

__attribute__((target("avx2,fma,f16c")))
static float q4q8_avx2(size_t blocks, const uint8_t *w, const int8_t *q, const float *d, const int16_t *bs) {
    float acc = 0.0f;
    const __m128i m4 = _mm_set1_epi8(0x0F);
    for (size_t i = 0; i < blocks; i++, w += 18, q += 32, bs += 2) {
        __m128i qs = _mm_loadu_si128((const __m128i *)(w + 2));
        __m256i codes = _mm256_set_m128i(_mm_and_si128(_mm_srli_epi16(qs, 4), m4), _mm_and_si128(qs, m4));
        int32_t s = hsum_epi32(dot_u8s8(codes, _mm256_loadu_si256((const __m256i *)q)));
        int32_t isum = s - 8 * ((int32_t)bs[0] + (int32_t)bs[1]); /* q4Corrections, cpu_quant_q8.go:314-322 */
        float t = trq_f16_to_f32((uint16_t)(w[0] | (w[1] << 8))) * d[i];
        acc = acc + t * (float)isum;
    }
    return acc;
}

void trq_avx2_quant_gemm_act(int dt, size_t M, size_t N, size_t K, const float *a,
                             const uint8_t *w, float *c, int threads) {
    if (K == 0 || M == 0 || N == 0) return;
    if (threads < 1) threads = 1;
    int blk = trq_block_elems(dt);
    size_t nb = K / (size_t)blk, rb = K / (size_t)blk * (size_t)trq_block_bytes(dt);
    int8_t *q = (int8_t *)malloc(M * K + 1);
    float *d = (float *)malloc(M * nb * sizeof(float) + 4);
    int16_t *bs = (int16_t *)malloc(M * (K / 16) * sizeof(int16_t) + 2);
    char *finite = (char *)malloc(M + 1);
    for (size_t m = 0; m < M; m++) {
        const float *r = a + m * K;
        int ok = 1;
        for (size_t k = 0; k < K; k++)
            if ((r[k] - r[k]) != 0.0f) { ok = 0; break; }
        finite[m] = (char)ok;
    }
#pragma omp parallel for num_threads(threads) schedule(guided)
    for (long m = 0; m < (long)M; m++)
        if (finite[m]) trq_quantize_q8(a + (size_t)m * K, K, blk, q + (size_t)m * K, d + (size_t)m * nb, bs + (size_t)m * (K / 16));
    for (size_t m = 0; m < M; m++)
        if (!finite[m]) trq_avx2_quant_gemv(dt, N, K, a + m * K, w, c + m * N, threads);
    /* work unit: 16 weight rows x all activation rows (q8BlockN, cpu_quant_q8.go:341) */
    const size_t unit = 16;
#pragma omp parallel for num_threads(threads) schedule(guided)
    for (long u = 0; u < (long)((N + unit - 1) / unit); u++) {
        size_t n0 = (size_t)u * unit, n1 = n0 + unit < N ? n0 + unit : N;
        for (size_t m = 0; m < M; m++) {
            if (!finite[m]) continue;
            const int8_t *qm = q + m * K;
            const float *dm = d + m * nb;
            const int16_t *bm = bs + m * (K / 16);
            for (size_t n = n0; n < n1; n++) {
                const uint8_t *wr = w + n * rb;
                float v = dt == TRQ_Q4K ? q4kq8_avx2(nb, wr, qm, dm, bm)
                        : dt == TRQ_Q6K ? q6kq8_avx2(nb, wr, qm, dm, bm)
                                        : q4q8_avx2(nb, wr, qm, dm, bm);
                c[m * N + n] = c[m * N + n] + v;
            }
        }
    }
    free(q);
    free(d);
    free(bs);
    free(finite);
}
