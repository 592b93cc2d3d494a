// wstore.hip -- weight-store repack/unpack, OpenQuant (dequant) and quantized embedding.
//
// The repack is a pure byte permutation of GGUF blocks into planes (layout in
// trhip_internal.hpp); unpack is its inverse (RawBackend.ToRaw, tensor/typed.go:27).
// Dequantization is bit-identical to tensor/quant.go:139-205: every product the reference
// keeps exact stays exact here and every rounding happens at the same operation (the file is
// compiled with -ffp-contract=off, so no multiply-add is fused unless written as fmaf).
#include "trhip_internal.hpp"

namespace trhip {
namespace {

// Destination offset of byte `i` of a q4_k qs block (lane slicing) and of q6_k ql/qh.
__host__ __device__ inline int q6k_ql_dst(int i) {  // old = 64n + 32h + 8t + l -> 32t + 16n + 8h + l
    int n = i >> 6, h = (i >> 5) & 1, t = (i >> 3) & 3, l = i & 7;
    return 32 * t + 16 * n + 8 * h + l;
}
__host__ __device__ inline int q6k_qh_dst(int i) {  // old = 32n + 8t + l -> 16t + 8n + l
    int n = i >> 5, t = (i >> 3) & 3, l = i & 7;
    return 16 * t + 8 * n + l;
}

template <int DT>
__global__ void repack_kernel(const uint8_t *__restrict__ raw, uint8_t *__restrict__ qs, uint8_t *__restrict__ aux,
                              uint8_t *__restrict__ sc, uint16_t *__restrict__ d, int64_t nblocks, bool inverse) {
    int64_t bi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (bi >= nblocks) return;
    uint8_t *rb = const_cast<uint8_t *>(raw) + bi * block_bytes(DT);
    uint8_t *q = qs + bi * qs_bytes(DT);
    // `inverse` swaps source and destination of every byte move.
    auto mv = [&](uint8_t *plane_byte, uint8_t *raw_byte) {
        if (inverse) *raw_byte = *plane_byte; else *plane_byte = *raw_byte;
    };
    if (DT == kQ8 || DT == kQ4) {
        uint8_t *dd = reinterpret_cast<uint8_t *>(d + bi);
        mv(dd, rb);
        mv(dd + 1, rb + 1);
        for (int i = 0; i < qs_bytes(DT); i++) mv(q + i, rb + 2 + i);
    } else if (DT == kQ4K) {
        uint8_t *h = aux + bi * 16;
        for (int i = 0; i < 16; i++) mv(h + i, rb + i);
        for (int i = 0; i < 128; i++) mv(q + q4k_pos(i), rb + 16 + i);
    } else {  // q6_k: ql[128] qh[64] sc[16] d[2]
        uint8_t *h = aux + bi * 64, *s = sc + bi * 16;
        uint8_t *dd = reinterpret_cast<uint8_t *>(d + bi);
        for (int i = 0; i < 128; i++) mv(q + q6k_ql_dst(i), rb + i);
        for (int i = 0; i < 64; i++) mv(h + q6k_qh_dst(i), rb + 128 + i);
        for (int i = 0; i < 16; i++) mv(s + i, rb + 192 + i);
        mv(dd, rb + 208);
        mv(dd + 1, rb + 209);
    }
}

// Dequantize 32 consecutive elements (one 32-element group) per thread; tensor/quant.go:139-205.
template <int DT>
__device__ void dequant_group(const Planes p, int64_t bi, int G, float *y) {
    if (DT == kQ8) {
        float d = f16_to_f32(p.d[bi]);
        const int8_t *c = reinterpret_cast<const int8_t *>(p.qs + bi * 32);
        for (int j = 0; j < 32; j++) y[j] = (float)c[j] * d;
    } else if (DT == kQ4) {
        float d = f16_to_f32(p.d[bi]);
        const uint8_t *c = p.qs + bi * 16;
        // group G of a q4 block is the whole block (32 elements)
        for (int j = 0; j < 16; j++) {
            y[j] = (float)((int)(c[j] & 0xF) - 8) * d;
            y[j + 16] = (float)((int)(c[j] >> 4) - 8) * d;
        }
    } else if (DT == kQ4K) {
        const uint8_t *h = p.aux + bi * 16;
        float d = f16_to_f32((uint16_t)(h[0] | (h[1] << 8)));
        float dmin = f16_to_f32((uint16_t)(h[2] | (h[3] << 8)));
        const uint8_t *s = h + 4;
        int j = G;  // sub-block j: low nibbles of group j/2 for even j, high nibbles for odd j
        uint8_t scv, mv;
        if (j < 4) {
            scv = s[j] & 63;
            mv = s[j + 4] & 63;
        } else {
            scv = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
            mv = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
        }
        float d1 = d * (float)scv, m1 = dmin * (float)mv;
        const uint8_t *q = p.qs + bi * 128;
        int g = j >> 1;
        for (int e = 0; e < 32; e++) {
            uint8_t b = q[q4k_pos(32 * g + e)];  // old byte 32g + e
            uint32_t code = (j & 1) ? (b >> 4) : (b & 0xF);
            y[e] = d1 * (float)code - m1;
        }
    } else {  // q6_k, 32-element group G = 4n + k: elements 128n + 32k + e
        float d = f16_to_f32(p.d[bi]);
        const int8_t *sc = reinterpret_cast<const int8_t *>(p.sc + bi * 16);
        const uint8_t *ql = p.qs + bi * 128, *qh = p.aux + bi * 64;
        int n = G >> 2, k = G & 3;
        for (int e = 0; e < 32; e++) {
            int t = e >> 3, l = e & 7;
            uint8_t lo = ql[32 * t + 16 * n + 8 * (k & 1) + l];
            uint8_t hb = qh[16 * t + 8 * n + l];
            int nib = (k < 2) ? (lo & 0xF) : (lo >> 4);
            int code = nib | (((hb >> (2 * k)) & 3) << 4);
            int is = e / 16;
            y[e] = d * (float)sc[8 * n + is + 2 * k] * (float)(code - 32);
        }
    }
}

template <int DT>
__global__ void dequant_kernel(const Planes p, int64_t block0, int64_t ngroups, float *__restrict__ out) {
    int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= ngroups) return;
    constexpr int per = block_elems(DT) / 32;
    int64_t bi = block0 + gi / per;
    int G = (int)(gi % per);
    float y[32];
    dequant_group<DT>(p, bi, G, y);
    float4 *o = reinterpret_cast<float4 *>(out + gi * 32);
    for (int i = 0; i < 8; i++) o[i] = make_float4(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
}

template <int DT>
__global__ void embedding_kernel(const Planes p, int64_t N, const int64_t *__restrict__ idx, int64_t nidx,
                                 float *__restrict__ out) {
    constexpr int per = block_elems(DT) / 32;
    int64_t groups_per_row = p.nb * per;
    int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= nidx * groups_per_row) return;
    int64_t i = gi / groups_per_row, gr = gi % groups_per_row;
    int64_t r = idx[i];
    float y[32];
    dequant_group<DT>(p, r * p.nb + gr / per, (int)(gr % per), y);
    float4 *o = reinterpret_cast<float4 *>(out + gi * 32);
    for (int k = 0; k < 8; k++) o[k] = make_float4(y[4 * k], y[4 * k + 1], y[4 * k + 2], y[4 * k + 3]);
}

template <template <int> class F, typename... A>
int dispatch_dt(int dt, A... a) {
    switch (dt) {
    case kQ8: return F<kQ8>::run(a...);
    case kQ4: return F<kQ4>::run(a...);
    case kQ4K: return F<kQ4K>::run(a...);
    case kQ6K: return F<kQ6K>::run(a...);
    }
    return TRHIP_ERR_INVALID;
}

template <int DT>
struct RepackRun {
    static int run(trhip_ctx *ctx, const trhip_wstore *w, uint8_t *raw, int64_t block0, int64_t nblocks, bool inv) {
        if (nblocks == 0) return TRHIP_OK;
        const int threads = 256;
        int64_t grid = (nblocks + threads - 1) / threads;
        hipLaunchKernelGGL(repack_kernel<DT>, dim3((unsigned)grid), dim3(threads), 0, ctx->stream, raw,
                           w->qs + block0 * qs_bytes(DT), w->aux ? w->aux + block0 * aux_bytes(DT) : nullptr,
                           w->sc ? w->sc + block0 * sc_bytes(DT) : nullptr, w->d ? w->d + block0 : nullptr, nblocks,
                           inv);
        return launch_check(ctx, inv ? "unpack" : "repack");
    }
};

template <int DT>
struct DequantRun {
    static int run(trhip_ctx *ctx, const trhip_wstore *w, int64_t block0, int64_t nblocks, float *out) {
        int64_t ngroups = nblocks * (block_elems(DT) / 32);
        if (ngroups == 0) return TRHIP_OK;
        const int threads = 256;
        hipLaunchKernelGGL(dequant_kernel<DT>, dim3((unsigned)((ngroups + threads - 1) / threads)), dim3(threads), 0,
                           ctx->stream, w->planes(), block0, ngroups, out);
        return launch_check(ctx, "open_q");
    }
};

template <int DT>
struct EmbedRun {
    static int run(trhip_ctx *ctx, const trhip_wstore *w, const int64_t *idx, int64_t nidx, float *out) {
        int64_t total = nidx * w->nb * (block_elems(DT) / 32);
        if (total == 0) return TRHIP_OK;
        const int threads = 256;
        hipLaunchKernelGGL(embedding_kernel<DT>, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0,
                           ctx->stream, w->planes(), w->N, idx, nidx, out);
        return launch_check(ctx, "embedding_q");
    }
};

}  // namespace

int launch_repack(trhip_ctx *ctx, trhip_wstore *w, const uint8_t *raw_dev) {
    return dispatch_dt<RepackRun>(w->dtype, ctx, (const trhip_wstore *)w, const_cast<uint8_t *>(raw_dev), (int64_t)0,
                                  w->N * w->nb, false);
}

int launch_unpack(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t rows, uint8_t *raw_dev) {
    return dispatch_dt<RepackRun>(w->dtype, ctx, w, raw_dev, row0 * w->nb, rows * w->nb, true);
}

int launch_dequant(trhip_ctx *ctx, const trhip_wstore *w, int64_t block0, int64_t nblocks, float *out) {
    return dispatch_dt<DequantRun>(w->dtype, ctx, w, block0, nblocks, out);
}

int launch_embedding(trhip_ctx *ctx, const trhip_wstore *w, const int64_t *idx, int64_t nidx, float *out,
                     int *bad_dev) {
    (void)bad_dev;
    return dispatch_dt<EmbedRun>(w->dtype, ctx, w, idx, nidx, out);
}

}  // namespace trhip
