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

// Elements 4f .. 4f+3 of block bi, dequantized as tensor/quant.go:139-205 (one thread per four outputs, so a
// wave's stores cover 1 KB of contiguous output). Every code word is one aligned dword of its plane: the four
// elements share their scale and min, and their bytes are contiguous in the repacked planes.
template <int DT>
__device__ __forceinline__ float4 dequant4(const Planes p, int64_t bi, int f) {
    const int e = 4 * f;
    float y[4];
    if (DT == kQ8) {
        const float d = f16_to_f32(p.d[bi]);
        const uint32_t c = *reinterpret_cast<const uint32_t *>(p.qs + bi * 32 + e);
#pragma unroll
        for (int k = 0; k < 4; k++) y[k] = (float)(int8_t)((c >> (8 * k)) & 0xFF) * d;
    } else if (DT == kQ4) {  // element j < 16: low nibble of byte j; j >= 16: high nibble of byte j - 16
        const float d = f16_to_f32(p.d[bi]);
        const uint32_t c = *reinterpret_cast<const uint32_t *>(p.qs + bi * 16 + (e & 15));
        const int sh = e < 16 ? 0 : 4;
#pragma unroll
        for (int k = 0; k < 4; k++) y[k] = (float)((int)((c >> (8 * k + sh)) & 0xF) - 8) * d;
    } else if (DT == kQ4K) {  // sub-block j = e / 32: low nibbles of group j / 2 for even j, high for odd j
        const uint4 h = *reinterpret_cast<const uint4 *>(p.aux + bi * 16);  // d, dmin, scales[12]
        const float d = f16_to_f32((uint16_t)(h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(h.x >> 16));
        const int j = e >> 5, g = e >> 6, ee = e & 31;
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(h.y, h.z, h.w, sc_lo, sc_hi, m_lo, m_hi);
        const float scv = ubyte_f(j < 4 ? sc_lo : sc_hi, j & 3), mv = ubyte_f(j < 4 ? m_lo : m_hi, j & 3);
        const float d1 = d * scv, m1 = dmin * mv;
        const uint32_t c = *reinterpret_cast<const uint32_t *>(p.qs + bi * 128 + q4k_pos(32 * g + ee));
        const int sh = (j & 1) ? 4 : 0;
#pragma unroll
        for (int k = 0; k < 4; k++) y[k] = d1 * (float)((c >> (8 * k + sh)) & 0xF) - m1;
    } else {  // q6_k, 32-element group k4 of half n: elements 128n + 32k4 + ee
        const float d = f16_to_f32(p.d[bi]);
        const int n = e >> 7, k4 = (e >> 5) & 3, ee = e & 31, t = ee >> 3, l = ee & 7;
        const uint32_t lo = *reinterpret_cast<const uint32_t *>(p.qs + bi * 128 + 32 * t + 16 * n + 8 * (k4 & 1) + l);
        const uint32_t hb = *reinterpret_cast<const uint32_t *>(p.aux + bi * 64 + 16 * t + 8 * n + l);
        const float sc = (float)(int8_t)p.sc[bi * 16 + 8 * n + 2 * k4 + ee / 16];
        const int sh = k4 < 2 ? 0 : 4;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int code = (int)((lo >> (8 * k + sh)) & 0xF) | (int)(((hb >> (8 * k + 2 * k4)) & 3) << 4);
            y[k] = d * sc * (float)(code - 32);
        }
    }
    return make_float4(y[0], y[1], y[2], y[3]);
}

// out may be any float pointer: aligned outputs take one 16-byte store, others four 4-byte stores
__device__ __forceinline__ void store4(float *out, int64_t i, float4 v, bool aligned) {
    if (aligned) {
        reinterpret_cast<float4 *>(out)[i] = v;
    } else {
        out[4 * i] = v.x;
        out[4 * i + 1] = v.y;
        out[4 * i + 2] = v.z;
        out[4 * i + 3] = v.w;
    }
}

template <int DT>
__global__ void dequant_kernel(const Planes p, int64_t block0, int64_t n4, float *__restrict__ out, bool aligned) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    constexpr int per = block_elems(DT) / 4;
    store4(out, i, dequant4<DT>(p, block0 + i / per, (int)(i % per)), aligned);
}

template <int DT>
__global__ void embedding_kernel(const Planes p, const int64_t *__restrict__ idx, int64_t nidx,
                                 float *__restrict__ out, bool aligned) {
    constexpr int per = block_elems(DT) / 4;
    const int64_t row4 = p.nb * per;  // float4 per output row
    const int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gi >= nidx * row4) return;
    const int64_t i = gi / row4, f = gi % row4;
    store4(out, gi, dequant4<DT>(p, idx[i] * p.nb + f / per, (int)(f % per)), aligned);
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
        const int64_t n4 = nblocks * (block_elems(DT) / 4);
        if (n4 == 0) return TRHIP_OK;
        const int threads = 256;
        if ((n4 + threads - 1) / threads >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "open_q: too many elements");
        hipLaunchKernelGGL(dequant_kernel<DT>, dim3((unsigned)((n4 + threads - 1) / threads)), dim3(threads), 0,
                           ctx->stream, w->planes(), block0, n4, out, reinterpret_cast<uintptr_t>(out) % 16 == 0);
        return launch_check(ctx, "open_q");
    }
};

template <int DT>
struct EmbedRun {
    static int run(trhip_ctx *ctx, const trhip_wstore *w, const int64_t *idx, int64_t nidx, float *out) {
        const int64_t total = nidx * w->nb * (block_elems(DT) / 4);
        if (total == 0) return TRHIP_OK;
        const int threads = 256;
        if ((total + threads - 1) / threads >= ((int64_t)1 << 31))
            return fail(ctx, TRHIP_ERR_UNSUPPORTED, "embedding_q: too many elements");
        hipLaunchKernelGGL(embedding_kernel<DT>, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0,
                           ctx->stream, w->planes(), idx, nidx, out, reinterpret_cast<uintptr_t>(out) % 16 == 0);
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
