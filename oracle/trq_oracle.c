/*
 * trq_oracle.c -- scalar C restatement of TR's CPU quantized matmul (test infrastructure).
 *
 * Built with -O2 -ffp-contract=off: every float operation below rounds on its own, and the
 * reference's fused multiply-adds are written as explicit fmaf() calls at exactly the
 * places where the reference's assembly uses VFMADD231PS / VFMSUB213PS.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this code, and
 * only as the expected result or the timed CPU baseline; the product library never calls it.
 */
#include "trq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int trq_block_elems(int dt) {
    switch (dt) {
    case TRQ_Q8: case TRQ_Q4: return 32;
    case TRQ_Q4K: case TRQ_Q6K: return 256;
    }
    return 0;
}

int trq_block_bytes(int dt) { /* quant.go:23-29 */
    switch (dt) {
    case TRQ_Q8: return 34;
    case TRQ_Q4: return 18;
    case TRQ_Q4K: return 144;
    case TRQ_Q6K: return 210;
    }
    return 0;
}

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* cpu_dtype.go:126-145 */
float trq_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    if (e == 0x1F) return bits_f32(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        uint32_t ex = 127 - 14;
        while ((m & 0x400) == 0) { m <<= 1; ex--; }
        return bits_f32(sign | (ex << 23) | ((m & 0x3FF) << 13));
    }
    return bits_f32(sign | ((e + 127 - 15) << 23) | (m << 13));
}

static float fp16(const uint8_t *p) { return trq_f16_to_f32(le16(p)); } /* quant.go:136 */

/* 16-bit activations and outputs (the typed matmul): cpu_dtype.go:73-80 (f32ToBF16), :83 (bf16ToF32), :87-123
 * (f32ToF16), :125-145 (f16ToF32, trq_f16_to_f32 above). type 1 = f16, 2 = bf16. */
static uint16_t f32_to_bf16(float f) {
    uint32_t b = f32_bits(f);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x0040u); /* NaN, quieted */
    b += 0x7FFFu + ((b >> 16) & 1u);                                            /* to nearest even */
    return (uint16_t)(b >> 16);
}

static uint16_t f32_to_f16(float f) {
    const uint32_t b = f32_bits(f);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    const int ex = (int)((b >> 23) & 0xFFu);
    uint32_t man = b & 0x7FFFFFu;
    if (ex == 0xFF) return man ? (uint16_t)(sign | 0x7E00u | (man >> 13)) : (uint16_t)(sign | 0x7C00u);
    const int e = ex - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) { /* subnormal or zero: the significand with its hidden bit, shifted */
        if (e < -10) return sign;
        man |= 0x800000u;
        const unsigned sh = (unsigned)(14 - e);
        uint32_t q = man >> sh;
        const uint32_t rest = man & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rest > half || (rest == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rest = man & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

void trq_round16(int type, const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = type == 2 ? f32_to_bf16(src[i]) : f32_to_f16(src[i]);
}

void trq_widen16(int type, const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = type == 2 ? bits_f32((uint32_t)src[i] << 16) : trq_f16_to_f32(src[i]);
}

/* quant.go:158-163 */
void trq_q4k_scale(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* quant.go:139-144 */
static void dequant_q8(float *y, const uint8_t *b) {
    float d = fp16(b);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}

/* quant.go:149-155 */
static void dequant_q4(float *y, const uint8_t *b) {
    float d = fp16(b);
    for (int j = 0; j < 16; j++) {
        uint8_t q = b[2 + j];
        y[j] = (float)((int)(q & 0xF) - 8) * d;
        y[j + 16] = (float)((int)(q >> 4) - 8) * d;
    }
}

/* quant.go:167-182: products exact, one rounding in the subtraction. */
static void dequant_q4k(float *y, const uint8_t *b) {
    float d = fp16(b), dmin = fp16(b + 2);
    const uint8_t *scales = b + 4, *q = b + 16;
    for (int g = 0; g < 4; g++) {
        uint8_t sc, m;
        trq_q4k_scale(2 * g, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        trq_q4k_scale(2 * g + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = dmin * (float)m;
        float *row = y + g * 64;
        for (int l = 0; l < 32; l++) {
            row[l] = d1 * (float)(q[l] & 0xF) - m1;
            row[l + 32] = d2 * (float)(q[l] >> 4) - m2;
        }
        q += 32;
    }
}

/* quant.go:185-205: (d*sc) exact, the product with (code-32) may round. */
static void dequant_q6k(float *y, const uint8_t *b) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = fp16(b + 208);
    for (int n = 0; n < 2; n++) {
        float *row = y + n * 128;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            uint8_t h = qh[l];
            int q1 = (int)((ql[l] & 0xF) | ((h & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
            row[l] = d * (float)sc[is] * (float)q1;
            row[l + 32] = d * (float)sc[is + 2] * (float)q2;
            row[l + 64] = d * (float)sc[is + 4] * (float)q3;
            row[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

/* quant.go:207-221 */
void trq_dequant(int dt, const uint8_t *raw, size_t nblocks, float *y) {
    int elems = trq_block_elems(dt), size = trq_block_bytes(dt);
    for (size_t i = 0; i < nblocks; i++) {
        const uint8_t *b = raw + i * (size_t)size;
        float *o = y + i * (size_t)elems;
        switch (dt) {
        case TRQ_Q8: dequant_q8(o, b); break;
        case TRQ_Q4: dequant_q4(o, b); break;
        case TRQ_Q4K: dequant_q4k(o, b); break;
        case TRQ_Q6K: dequant_q6k(o, b); break;
        }
    }
}

/* quant.go:130-133 */
static int bad_scale(const uint8_t *p) { return (le16(p) & 0x7C00) == 0x7C00; }

/* quant.go:108-128 */
long trq_check_quant_scales(int dt, const uint8_t *raw, size_t nbytes) {
    size_t size = (size_t)trq_block_bytes(dt);
    for (size_t b = 0; b * size < nbytes; b++) {
        const uint8_t *blk = raw + b * size;
        int bad = 0;
        switch (dt) {
        case TRQ_Q8: case TRQ_Q4: bad = bad_scale(blk); break;
        case TRQ_Q4K: bad = bad_scale(blk) || bad_scale(blk + 2); break;
        case TRQ_Q6K: bad = bad_scale(blk + 208); break;
        }
        if (bad) return (long)b;
    }
    return -1;
}

/* quant.go:416-427 */
void trq_quant_zero_raw(int dt, size_t n, uint8_t *out) {
    size_t size = (size_t)trq_block_bytes(dt), blocks = n / (size_t)trq_block_elems(dt);
    memset(out, 0, blocks * size);
    if (dt == TRQ_Q4)
        for (size_t b = 0; b < blocks; b++) memset(out + b * size + 2, 0x88, size - 2);
}

/* cpu_gemv.go:66-85 (dot32): eight accumulators, no fusion (GOAMD64=v1 code generation). */
static float dot32(const float *x, const float *y, size_t n) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) s[l] = s[l] + x[i + l] * y[i + l];
    for (; i < n; i++) s[0] = s[0] + x[i] * y[i];
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

/* cpu_gemv_amd64.s:190-227 (sdot32): element i is fused into accumulator (i/8)%4, lane i%8,
 * in ascending i; then Y=(A0+A1)+(A2+A3), s_l = Y[l]+Y[l+4], result (s0+s2)+(s1+s3). */
static float sdot32(const float *x, const float *y, size_t n) {
    float acc[32];
    for (int l = 0; l < 32; l++) acc[l] = 0.0f;
    for (size_t i = 0; i < n; i++) acc[i % 32] = fmaf(x[i], y[i], acc[i % 32]);
    float Y[8], s[4];
    for (int l = 0; l < 8; l++) Y[l] = (acc[l] + acc[8 + l]) + (acc[16 + l] + acc[24 + l]);
    for (int l = 0; l < 4; l++) s[l] = Y[l] + Y[l + 4];
    return (s[0] + s[2]) + (s[1] + s[3]);
}

/* cpu_gemv_amd64.go:25-35 (dotF32) on an AVX2 machine. */
float trq_dot_f32(const float *x, const float *y, size_t n) {
    if (n < 32) return dot32(x, y, n);
    size_t n32 = n & ~(size_t)31;
    float s = sdot32(x, y, n32);
    if (n32 < n) s = s + dot32(x + n32, y + n32, n - n32);
    return s;
}

/* cpu_quant.go:38-44 (dotQuantGo): dequant + dotF32, bit-identical to quantDot. */
float trq_quant_dot(int dt, const float *x, const uint8_t *w, size_t K) {
    float *row = (float *)malloc(K * sizeof(float) + 1);
    trq_dequant(dt, w, K / (size_t)trq_block_elems(dt), row);
    float s = trq_dot_f32(x, row, K);
    free(row);
    return s;
}

static size_t row_bytes(int dt, size_t K) { /* cpu_quant.go:21-24 */
    return K / (size_t)trq_block_elems(dt) * (size_t)trq_block_bytes(dt);
}

/* cpu_matmul.go:29 (kcBlock) */
#define KC_BLOCK 256

/* M>1 order shared by quantGemmPanels (cpu_quant.go:103-147) and the tile path
 * (cpu_quant.go:59-82 -> gemmPart, cpu_matmul.go:330-380): for each 256-deep K chunk
 * a fresh fused chain from +0 in ascending k (sgemm6x16, cpu_micro_amd64.s:14-64), the
 * chunk results added in order into a cleared part (VADDPS (DX) at :66-95), then c += part. */
static void gemm_rows_chunked(size_t M, size_t N, size_t K, const float *a, const float *wdeq,
                              float *c, size_t n0, size_t n1) {
    for (size_t n = n0; n < n1; n++) {
        const float *wr = wdeq + (n - n0) * K;
        for (size_t m = 0; m < M; m++) {
            const float *ar = a + m * K;
            float part = 0.0f;
            for (size_t p0 = 0; p0 < K; p0 += KC_BLOCK) {
                size_t kb = K - p0 < KC_BLOCK ? K - p0 : KC_BLOCK;
                float chain = 0.0f;
                for (size_t k = 0; k < kb; k++) chain = fmaf(ar[p0 + k], wr[p0 + k], chain);
                part = part + chain;
            }
            c[m * N + n] = c[m * N + n] + part;
        }
    }
}

/* cpu_quant.go:47-83 */
void trq_quant_gemm(int dt, size_t M, size_t N, size_t K, const float *a, const uint8_t *w,
                    float *c, int threads) {
    if (K == 0 || M == 0 || N == 0) return;
    size_t rb = row_bytes(dt, K), nb = K / (size_t)trq_block_elems(dt);
    if (threads < 1) threads = 1;
    if (M == 1) { /* quantGemv, cpu_quant.go:151-160 */
#pragma omp parallel num_threads(threads)
        {
            float *row = (float *)malloc(K * sizeof(float) + 1);
#pragma omp for schedule(guided)
            for (long n = 0; n < (long)N; n++) {
                trq_dequant(dt, w + (size_t)n * rb, nb, row);
                c[n] = c[n] + trq_dot_f32(a, row, K);
            }
            free(row);
        }
        return;
    }
    const size_t tile = 16;
#pragma omp parallel num_threads(threads)
    {
        float *rows = (float *)malloc(tile * K * sizeof(float) + 1);
#pragma omp for schedule(guided)
        for (long t = 0; t < (long)((N + tile - 1) / tile); t++) {
            size_t n0 = (size_t)t * tile, n1 = n0 + tile < N ? n0 + tile : N;
            trq_dequant(dt, w + n0 * rb, (n1 - n0) * nb, rows);
            gemm_rows_chunked(M, N, K, a, rows, c, n0, n1);
        }
        free(rows);
    }
}

/* cpu_quant_q8.go:39-68 */
void trq_quantize_q8(const float *x, size_t K, int blk, int8_t *q, float *d, int16_t *bs) {
    for (size_t b = 0; b < K / (size_t)blk; b++) {
        const float *v = x + b * (size_t)blk;
        int8_t *qb = q + b * (size_t)blk;
        float amax = 0.0f;
        for (int j = 0; j < blk; j++) {
            float a = fabsf(v[j]);
            if (a > amax) amax = a;
        }
        float id = 127.0f / amax;
        if (!(amax > 0.0f) || (id - id) != 0.0f) {
            memset(qb, 0, (size_t)blk);
            d[b] = 0.0f;
        } else {
            d[b] = amax / 127.0f;
            for (int j = 0; j < blk; j++) {
                float t = rintf(v[j] * id); /* RoundToEven(float64(float32(v*id))) */
                if (t > 127.0f) t = 127.0f;
                if (t < -127.0f) t = -127.0f;
                qb[j] = (int8_t)t;
            }
        }
        for (int s = 0; s < blk / 16; s++) {
            int16_t t = 0;
            for (int j = 0; j < 16; j++) t = (int16_t)(t + qb[s * 16 + j]);
            bs[b * (size_t)(blk / 16) + (size_t)s] = t;
        }
    }
}

/* cpu_quant_q8.go:74-87 */
float trq_dot_q4q8(size_t blocks, const uint8_t *w, const int8_t *q, const float *d) {
    float acc = 0.0f;
    for (size_t i = 0; i < blocks; i++) {
        const uint8_t *b = w + i * 18;
        const int8_t *a = q + i * 32;
        int32_t isum = 0;
        for (int j = 0; j < 16; j++)
            isum += ((int32_t)(b[2 + j] & 0xF) - 8) * a[j] + ((int32_t)(b[2 + j] >> 4) - 8) * a[j + 16];
        float t = fp16(b) * d[i];
        acc = acc + t * (float)isum;
    }
    return acc;
}

static void q4k_isums(const uint8_t *b, const int8_t *a, const int16_t *bs, int32_t *isum_out,
                      int32_t *msum_out) {
    const uint8_t *scales = b + 4, *q = b + 16;
    int32_t isum = 0, msum = 0;
    for (int g = 0; g < 4; g++) {
        uint8_t sc1, m1, sc2, m2;
        trq_q4k_scale(2 * g, scales, &sc1, &m1);
        trq_q4k_scale(2 * g + 1, scales, &sc2, &m2);
        int32_t s1 = 0, s2 = 0;
        for (int l = 0; l < 32; l++) {
            s1 += (int32_t)(q[l] & 0xF) * a[g * 64 + l];
            s2 += (int32_t)(q[l] >> 4) * a[g * 64 + 32 + l];
        }
        isum += (int32_t)sc1 * s1 + (int32_t)sc2 * s2;
        const int16_t *p = bs + g * 4;
        msum += (int32_t)m1 * (int32_t)(int16_t)(p[0] + p[1]) + (int32_t)m2 * (int32_t)(int16_t)(p[2] + p[3]);
        q += 32;
    }
    *isum_out = isum;
    *msum_out = msum;
}

/* cpu_quant_q8.go:91-116 */
float trq_dot_q4kq8(size_t blocks, const uint8_t *w, const int8_t *q, const float *d,
                    const int16_t *bs) {
    float acc = 0.0f;
    for (size_t i = 0; i < blocks; i++) {
        const uint8_t *b = w + i * 144;
        float dd = fp16(b), dmin = fp16(b + 2);
        int32_t isum, msum;
        q4k_isums(b, q + i * 256, bs + i * 16, &isum, &msum);
        float t = (dd * (float)isum) - (dmin * (float)msum);
        acc = acc + t * d[i];
    }
    return acc;
}

static int32_t q6k_isum(const uint8_t *b, const int8_t *a, const int16_t *bs) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    int32_t isum = 0, msum = 0;
    for (int n = 0; n < 2; n++) {
        for (int l = 0; l < 32; l++) {
            uint8_t h = qh[l];
            int32_t q1 = (ql[l] & 0xF) | ((h & 3) << 4);
            int32_t q2 = (ql[l + 32] & 0xF) | (((h >> 2) & 3) << 4);
            int32_t q3 = (ql[l] >> 4) | (((h >> 4) & 3) << 4);
            int32_t q4 = (ql[l + 32] >> 4) | (((h >> 6) & 3) << 4);
            int is = l / 16;
            isum += (int32_t)sc[is] * q1 * a[n * 128 + l] + (int32_t)sc[is + 2] * q2 * a[n * 128 + l + 32] +
                    (int32_t)sc[is + 4] * q3 * a[n * 128 + l + 64] + (int32_t)sc[is + 6] * q4 * a[n * 128 + l + 96];
        }
        ql += 64;
        qh += 32;
        sc += 8;
    }
    sc = (const int8_t *)(b + 192);
    for (int j = 0; j < 16; j++) msum += (int32_t)sc[j] * (int32_t)bs[j];
    return isum - 32 * msum;
}

/* cpu_quant_q8.go:378-407 */
float trq_dot_q6kq8(size_t blocks, const uint8_t *w, const int8_t *q, const float *d,
                    const int16_t *bs) {
    float acc = 0.0f;
    for (size_t i = 0; i < blocks; i++) {
        const uint8_t *b = w + i * 210;
        float dd = fp16(b + 208);
        int32_t v = q6k_isum(b, q + i * 256, bs + i * 16);
        float t = dd * (float)v;
        acc = acc + t * d[i];
    }
    return acc;
}

void trq_block_isums(int dt, size_t blocks, const uint8_t *w, const int8_t *q, const int16_t *bs,
                     int32_t *isum, int32_t *msum) {
    for (size_t i = 0; i < blocks; i++) {
        if (dt == TRQ_Q4) {
            const uint8_t *b = w + i * 18;
            const int8_t *a = q + i * 32;
            int32_t s = 0;
            for (int j = 0; j < 16; j++)
                s += ((int32_t)(b[2 + j] & 0xF) - 8) * a[j] + ((int32_t)(b[2 + j] >> 4) - 8) * a[j + 16];
            isum[i] = s;
            if (msum) msum[i] = 0;
        } else if (dt == TRQ_Q4K) {
            int32_t s, m;
            q4k_isums(w + i * 144, q + i * 256, bs + i * 16, &s, &m);
            isum[i] = s;
            if (msum) msum[i] = m;
        } else if (dt == TRQ_Q6K) {
            isum[i] = q6k_isum(w + i * 210, q + i * 256, bs + i * 16);
            if (msum) msum[i] = 0;
        }
    }
}

/* cpu_quant_q8.go:137-144 */
static int q8_finite(const float *a, size_t n) {
    for (size_t i = 0; i < n; i++)
        if ((a[i] - a[i]) != 0.0f || a[i] != a[i]) return 0;
    return 1;
}

static float dot_q8(int dt, size_t blocks, const uint8_t *w, const int8_t *q, const float *d,
                    const int16_t *bs) {
    switch (dt) {
    case TRQ_Q4: return trq_dot_q4q8(blocks, w, q, d);
    case TRQ_Q6K: return trq_dot_q6kq8(blocks, w, q, d, bs);
    }
    return trq_dot_q4kq8(blocks, w, q, d, bs);
}

/* cpu_quant_q8.go:125-134, :159-174, :186-259: every output element is one single-row
 * kernel result; non-finite rows go through quantGemv on their own. */
void trq_quant_gemm_act(int dt, size_t M, size_t N, size_t K, const float *a, const uint8_t *w,
                        float *c, int threads) {
    if (K == 0 || M == 0 || N == 0) return;
    if (threads < 1) threads = 1;
    int blk = trq_block_elems(dt);
    size_t nb = K / (size_t)blk, rb = row_bytes(dt, K);
    int8_t *q = (int8_t *)malloc(M * K + 1);
    float *d = (float *)malloc(M * nb * sizeof(float) + 4);
    int16_t *bs = (int16_t *)malloc(M * (K / 16) * sizeof(int16_t) + 2);
    char *finite = (char *)malloc(M + 1);
    for (size_t m = 0; m < M; m++) {
        finite[m] = (char)q8_finite(a + m * K, K);
        if (finite[m])
            trq_quantize_q8(a + m * K, K, blk, q + m * K, d + m * nb, bs + m * (K / 16));
        else
            trq_quant_gemm(dt, 1, N, K, a + m * K, w, c + m * N, threads);
    }
#pragma omp parallel for num_threads(threads) schedule(guided)
    for (long n = 0; n < (long)N; n++) {
        for (size_t m = 0; m < M; m++) {
            if (!finite[m]) continue;
            c[m * N + (size_t)n] = c[m * N + (size_t)n] +
                dot_q8(dt, nb, w + (size_t)n * rb, q + m * K, d + m * nb, bs + m * (K / 16));
        }
    }
    free(q);
    free(d);
    free(bs);
    free(finite);
}

/* cpu_quant.go:163-171 */
void trq_quant_embedding(int dt, const uint8_t *raw, size_t D, const int64_t *idx, size_t nidx,
                         float *out) {
    size_t rb = row_bytes(dt, D), nb = D / (size_t)trq_block_elems(dt);
    for (size_t i = 0; i < nidx; i++) trq_dequant(dt, raw + (size_t)idx[i] * rb, nb, out + i * D);
}

/* quant_test.go:20-46 */
void trq_random_quant(int dt, uint32_t seed, size_t blocks, uint8_t *raw) {
    size_t size = (size_t)trq_block_bytes(dt);
    uint32_t state = seed;
    for (size_t i = 0; i < blocks * size; i++) {
        state = state * 1664525u + 1013904223u;
        raw[i] = (uint8_t)(state >> 24);
    }
    for (size_t b = 0; b < blocks; b++) {
        uint8_t *blk = raw + b * size;
        int offs[2] = {0, -1};
        if (dt == TRQ_Q4K) offs[1] = 2;
        if (dt == TRQ_Q6K) offs[0] = 208;
        for (int k = 0; k < 2; k++) {
            if (offs[k] < 0) continue;
            uint8_t *p = blk + offs[k];
            uint16_t v = le16(p);
            if ((v & 0x7C00) == 0x7C00) {
                v = (uint16_t)(v & ~0x4000);
                p[0] = (uint8_t)v;
                p[1] = (uint8_t)(v >> 8);
            }
        }
    }
}

uint64_t trq_fnv1a64_f32(const float *y, size_t n) {
    uint64_t h = 14695981039346656037ull;
    for (size_t i = 0; i < n; i++) {
        uint32_t u = f32_bits(y[i]);
        for (int k = 0; k < 4; k++) {
            h ^= (uint8_t)(u >> (8 * k));
            h *= 1099511628211ull;
        }
    }
    return h;
}

/* ------------------------------------------------------------------ SwiGLU epilogue
 * e^x as the reference's AVX2 expVec computes it (cpu_vector_amd64.s:13-38, the UST macro, used by
 * expVec in cpu_vector_amd64.go:31-47 for every element, tail included): clamp to [-104, 89] (a NaN
 * input takes the lower bound and is put back at the end), n = rne(x * log2e), r = x - n*ln2 in two
 * fused steps, a degree-6 polynomial in fused steps, and 2^n applied as two factors 2^(n>>1) and
 * 2^(n - n>>1). The constants are the reference's (cpu_math.go:10-17, 43-50; the Cephes expf set). */
float trq_exp_vec(float x) {
    float x1 = x > -104.0f ? x : -104.0f;
    x1 = x1 < 89.0f ? x1 : 89.0f;
    const float n = rintf(x1 * 1.44269504088896341f);
    float r = fmaf(-n, 0.693359375f, x1);
    r = fmaf(-n, -2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    const float z = r * r;
    p = fmaf(z, p, r);
    float y = p + 1.0f;
    const int ni = (int)n, h = ni >> 1, l = ni - h;
    y = y * bits_f32((uint32_t)(h + 127) << 23);
    y = y * bits_f32((uint32_t)(l + 127) << 23);
    return x != x ? x : y;
}

/* x * sigma(x) as siluForward (cpu_elementwise_wide.go:101-116) with sigmoidBlock (:83-98):
 * e = e^-|x|, sigma = 1/(1+e) for x >= 0, e/(1+e) otherwise; sigma == 0 gives +0. */
float trq_silu(float x) {
    const float e = trq_exp_vec(-fabsf(x));
    const float s = x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    return (s == 0.0f ? 0.0f : x) * s;
}

/* swiglu_gate (lib/layers.tr:223): silu(g) * u on a [M, 2I] row-major [G | U] buffer
 * (the merged gate_up layout, layers.tr:240-262 and its .split(2)). */
void trq_swiglu(const float *gu, size_t M, size_t I, float *out) {
    for (size_t m = 0; m < M; m++)
        for (size_t i = 0; i < I; i++) out[m * I + i] = trq_silu(gu[m * 2 * I + i]) * gu[m * 2 * I + I + i];
}
