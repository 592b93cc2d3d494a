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

// Inverse maps: repacked position j of a q4_k qs / q6_k ql / q6_k qh byte -> its byte in the GGUF block field.
__host__ __device__ inline int q4k_src(int j) {  // j = 64a + 16g + 8h + l -> 32g + 16a + 8h + l
    return 32 * ((j >> 4) & 3) + 16 * (j >> 6) + (j & 15);
}
__host__ __device__ inline int q6k_ql_src(int j) {  // j = 32t + 16n + 8h + l -> 64n + 32h + 8t + l
    int t = j >> 5, n = (j >> 4) & 1, h = (j >> 3) & 1, l = j & 7;
    return 64 * n + 32 * h + 8 * t + l;
}
__host__ __device__ inline int q6k_qh_src(int j) {  // j = 16t + 8n + l -> 32n + 8t + l
    int t = j >> 4, n = (j >> 3) & 1, l = j & 7;
    return 32 * n + 8 * t + l;
}

// Fields of a GGUF block as planes (trhip_internal.hpp): plane k holds PB[k] bytes per block. Plane 0 is qs (q6_k ql),
// then aux (q4_k hdr, q6_k qh), sc, d, in that order for the planes a dtype has.
template <int DT>
struct Fields {
    static constexpr int NP = DT == kQ6K ? 4 : 2;
    static constexpr int pb(int k) {
        return DT == kQ8 ? (k == 0 ? 32 : 2)
             : DT == kQ4 ? (k == 0 ? 16 : 2)
             : DT == kQ4K ? (k == 0 ? 128 : 16)
                          : (k == 0 ? 128 : k == 1 ? 64 : k == 2 ? 16 : 2);
    }
    // GGUF block byte of plane k's byte j
    __device__ static int raw_of(int k, int j) {
        if (DT == kQ8 || DT == kQ4) return k == 0 ? 2 + j : j;
        if (DT == kQ4K) return k == 0 ? 16 + q4k_src(j) : j;
        return k == 0 ? q6k_ql_src(j) : k == 1 ? 128 + q6k_qh_src(j) : k == 2 ? 192 + j : 208 + j;
    }
    // plane and plane byte of GGUF block byte r
    __device__ static void plane_of(int r, int &k, int &j) {
        if (DT == kQ8 || DT == kQ4) { k = r < 2 ? 1 : 0; j = r < 2 ? r : r - 2; }
        else if (DT == kQ4K) { k = r < 16 ? 1 : 0; j = r < 16 ? r : q4k_pos(r - 16); }
        else if (r < 128) { k = 0; j = q6k_ql_dst(r); }
        else if (r < 192) { k = 1; j = q6k_qh_dst(r - 128); }
        else if (r < 208) { k = 2; j = r - 192; }
        else { k = 3; j = r - 208; }
    }
};

// LDS <- bytes of global memory: 16-byte loads where the source is aligned and whole, else byte loads. dst is
// 16-byte aligned.
__device__ __forceinline__ void load_lds(uint8_t *dst, const uint8_t *__restrict__ src, int bytes) {
    for (int u = threadIdx.x; 16 * u < bytes; u += blockDim.x) {
        const uint8_t *s = src + 16 * u;
        if (16 * u + 16 <= bytes && reinterpret_cast<uintptr_t>(s) % 16 == 0) {
            *reinterpret_cast<uint4 *>(dst + 16 * u) = *reinterpret_cast<const uint4 *>(s);
        } else {
            for (int k = 0; k < 16 && 16 * u + k < bytes; k++) dst[16 * u + k] = s[k];
        }
    }
}

// bytes [0, bytes) of dst <- a gather from LDS: byte o comes from lds[at(o)]. 16-byte stores where dst is aligned
// and the unit whole, else byte stores.
template <typename F>
__device__ __forceinline__ void store_gather(uint8_t *__restrict__ dst, int bytes, const uint8_t *lds, F at) {
    for (int u = threadIdx.x; 16 * u < bytes; u += blockDim.x) {
        uint8_t *d = dst + 16 * u;
        if (16 * u + 16 <= bytes && reinterpret_cast<uintptr_t>(d) % 16 == 0) {
            uint32_t wd[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                uint32_t v = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) v |= (uint32_t)lds[at(16 * u + 4 * q + k)] << (8 * k);
                wd[q] = v;
            }
            *reinterpret_cast<uint4 *>(d) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        } else {
            for (int k = 0; k < 16 && 16 * u + k < bytes; k++) d[k] = lds[at(16 * u + k)];
        }
    }
}

// Repack (GGUF blocks -> planes) or, with INV, unpack (planes -> GGUF blocks) of blocks [block0, block0 + nblocks)
// of a store; raw holds those blocks from its start. A workgroup takes RB consecutive blocks: it reads their source
// bytes into LDS with coalesced 16-byte loads and writes each destination region with coalesced 16-byte stores,
// gathering the bytes from LDS (a byte permutation, nothing is decoded).
constexpr int RB = 64;
template <int DT, bool INV>
__global__ __launch_bounds__(256) void repack_kernel(uint8_t *__restrict__ raw, uint8_t *__restrict__ qs,
                                                     uint8_t *__restrict__ aux, uint8_t *__restrict__ sc,
                                                     uint8_t *__restrict__ d, int64_t block0, int64_t nblocks) {
    using F = Fields<DT>;
    constexpr int BB = block_bytes(DT);
    __shared__ __align__(16) uint8_t lds[RB * BB + 64];
    const int64_t g0 = (int64_t)blockIdx.x * RB;  // first block of this workgroup, relative to block0
    const int nbk = (int)(nblocks - g0 < RB ? nblocks - g0 : RB);
    uint8_t *planes[4] = {qs, aux, sc, d};
    uint8_t *rg = raw + g0 * BB;
    if (!INV) {
        load_lds(lds, rg, nbk * BB);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < F::NP; k++) {
            const int pb = F::pb(k);
            store_gather(planes[k] + (block0 + g0) * pb, nbk * pb, lds,
                         [&](int o) { return (o / pb) * BB + F::raw_of(k, o % pb); });
        }
    } else {
        int base[4], at = 0;
#pragma unroll
        for (int k = 0; k < F::NP; k++) {  // plane sections of the group in LDS, each 16-byte aligned
            base[k] = at;
            load_lds(lds + at, planes[k] + (block0 + g0) * F::pb(k), nbk * F::pb(k));
            at += (nbk * F::pb(k) + 15) / 16 * 16;
        }
        __syncthreads();
        store_gather(rg, nbk * BB, lds, [&](int o) {
            int k, j;
            F::plane_of(o % BB, k, j);
            return base[k] + (o / BB) * F::pb(k) + j;
        });
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
        const int64_t grid = (nblocks + RB - 1) / RB;
        if (grid >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "repack: too many blocks");
        uint8_t *d8 = reinterpret_cast<uint8_t *>(w->d);
        uint8_t *p1 = DT == kQ8 || DT == kQ4 ? d8 : w->aux, *p2 = w->sc, *p3 = DT == kQ6K ? d8 : nullptr;
        if (inv)
            hipLaunchKernelGGL((repack_kernel<DT, true>), dim3((unsigned)grid), dim3(256), 0, ctx->stream, raw, w->qs,
                               p1, p2, p3, block0, nblocks);
        else
            hipLaunchKernelGGL((repack_kernel<DT, false>), dim3((unsigned)grid), dim3(256), 0, ctx->stream, raw, w->qs,
                               p1, p2, p3, block0, nblocks);
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

int launch_repack(trhip_ctx *ctx, trhip_wstore *w, const uint8_t *raw_dev, int64_t block0, int64_t nblocks) {
    return dispatch_dt<RepackRun>(w->dtype, ctx, (const trhip_wstore *)w, const_cast<uint8_t *>(raw_dev), block0,
                                  nblocks, false);
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
