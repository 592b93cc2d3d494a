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
// Latency hiding: x is staged once per workgroup in LDS; each lane keeps a ring of DEPTH blocks of
// weight bytes in registers and issues the loads for block b+DEPTH before it computes block b, so every
// wave has DEPTH blocks of HBM reads in flight. Every weight byte is read exactly once.
#include "trhip_internal.hpp"

#include <cstdlib>
#include <type_traits>

namespace trhip {
namespace {

// Stage n float4 of x into LDS with THREADS threads, a batch of U float4 per thread at a time. issue() requests a
// batch (clamped, unconditional loads); commit() stores it. The empty asm on every loaded value keeps the loads
// ahead of it: without it the compiler moves each load into its store's branch, and a wait follows each one.
// A kernel issues the first batch, then its weight loads, then commits, so x and the first weights are in
// flight together and the wait before the stores covers x only.
// IO: fp32 x, or f16 / bf16 x read 8 bytes at a time and widened exactly on the way into LDS.
template <int THREADS, int IO = TRHIP_F32>
struct XStager {
    static constexpr int U = 8;
    typedef typename std::conditional<IO == TRHIP_F32, float4, uint2>::type Raw;
    Raw v[U];
    __device__ __forceinline__ void issue(const void *__restrict__ xv, int64_t n, int64_t i0) {
        const Raw *x4 = static_cast<const Raw *>(xv);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = i0 + (int64_t)u * THREADS + threadIdx.x;
            v[u] = x4[i < n ? i : n - 1];
        }
    }
    __device__ __forceinline__ void commit(float4 *xs, int64_t n, int64_t i0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            float4 f;
            if constexpr (IO == TRHIP_F32) {
                asm volatile("" : "+v"(v[u].x), "+v"(v[u].y), "+v"(v[u].z), "+v"(v[u].w));
                f = v[u];
            } else {
                asm volatile("" : "+v"(v[u].x), "+v"(v[u].y));
                f = make_float4(h16_to_f32(v[u].x & 0xFFFFu, IO), h16_to_f32(v[u].x >> 16, IO),
                                h16_to_f32(v[u].y & 0xFFFFu, IO), h16_to_f32(v[u].y >> 16, IO));
            }
            const int64_t i = i0 + (int64_t)u * THREADS + threadIdx.x;
            if (i < n) xs[i] = f;
        }
    }
    // the batches after the first
    __device__ __forceinline__ void rest(float4 *xs, const void *__restrict__ xv, int64_t n) {
        for (int64_t i0 = (int64_t)U * THREADS; i0 < n; i0 += (int64_t)U * THREADS) {
            issue(xv, n, i0);
            commit(xs, n, i0);
        }
    }
};

// c[r] (+)= res: fp32, or 16-bit c widened, the fp32 sum, rounded once
template <bool ACC, int IO>
__device__ __forceinline__ void put_out(void *cv, int64_t r, float res) {
    if constexpr (IO == TRHIP_F32) {
        float *c = static_cast<float *>(cv);
        c[r] = ACC ? c[r] + res : res;
    } else {
        uint16_t *c = static_cast<uint16_t *>(cv);
        c[r] = (uint16_t)f32_to_h16(ACC ? h16_to_f32(c[r], IO) + res : res, IO);
    }
}

__device__ __forceinline__ void fma4(float *acc, uint32_t codes, float s, float negm, float4 xv) {
    codes = opaque(codes);
    acc[0] = fmaf(fmaf(s, ubyte_f(codes, 0), negm), xv.x, acc[0]);
    acc[1] = fmaf(fmaf(s, ubyte_f(codes, 1), negm), xv.y, acc[1]);
    acc[2] = fmaf(fmaf(s, ubyte_f(codes, 2), negm), xv.z, acc[2]);
    acc[3] = fmaf(fmaf(s, ubyte_f(codes, 3), negm), xv.w, acc[3]);
}

// One 32-element group for this lane: 8 codes (two dwords), value = fmaf(s, code, negm); x from LDS.
__device__ __forceinline__ void group8(float *acc, uint32_t c0, uint32_t c1, float s, float negm,
                                       const float4 *xg) {
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

// Per-dtype block access. Data holds one block's bytes for one lane; load() fetches block b of the
// lane's row; compute() advances the lane's eight chains over that block. xb points at the LDS copy
// of x, at float4 index 2t of the block's first element.
template <int DT>
struct Blk;

template <>
struct Blk<kQ8> {
    static constexpr int DEPTH = 16;
    struct Data { uint2 q; uint32_t d; };
    const uint2 *qp;
    const uint16_t *dp;
    __device__ Blk(const Planes &p, int64_t row, int t)
        : qp(reinterpret_cast<const uint2 *>(p.qs + row * p.nb * 32) + t), dp(p.d + row * p.nb) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const { v.q = qp[4 * b]; v.d = dp[b]; }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb, int t) const {
        float d = f16_to_f32((uint16_t)v.d);
        // code = u - 128 with u = byte ^ 0x80; (u-128)*d is exact, so fmaf(d, u, -128d) is too
        group8(acc, v.q.x ^ 0x80808080u, v.q.y ^ 0x80808080u, d, -128.0f * d, xb);
    }
    static constexpr int XSTEP = 8;  // float4s of x per block
};

template <>
struct Blk<kQ4> {
    static constexpr int DEPTH = 16;
    struct Data { uint2 q; uint32_t d; };
    const uint2 *qp;
    const uint16_t *dp;
    int sh;
    __device__ Blk(const Planes &p, int64_t row, int t)
        : qp(reinterpret_cast<const uint2 *>(p.qs + row * p.nb * 16) + (t & 1)), dp(p.d + row * p.nb),
          sh((t & 2) ? 4 : 0) {}  // lanes 2,3 take the high nibbles (elements 16..31)
    __device__ __forceinline__ void load(Data &v, int64_t b) const { v.q = qp[2 * b]; v.d = dp[b]; }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb, int t) const {
        float d = f16_to_f32((uint16_t)v.d);
        group8(acc, (v.q.x >> sh) & 0x0F0F0F0Fu, (v.q.y >> sh) & 0x0F0F0F0Fu, d, -8.0f * d, xb);
    }
    static constexpr int XSTEP = 8;
};

template <>
struct Blk<kQ4K> {
    static constexpr int DEPTH = 6;
    struct Data { uint4 h; uint2 q[4]; };
    const uint4 *hp;
    const uint2 *qp;  // lane t's piece of group g sits at byte 64(t>>1) + 16g + 8(t&1) of the block
    __device__ Blk(const Planes &p, int64_t row, int t)
        : hp(reinterpret_cast<const uint4 *>(p.aux + row * p.nb * 16)),
          qp(reinterpret_cast<const uint2 *>(p.qs + row * p.nb * 128) + 8 * (t >> 1) + (t & 1)) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const {
        v.h = hp[b];
#pragma unroll
        for (int g = 0; g < 4; g++) v.q[g] = qp[16 * b + 2 * g];
    }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb, int t) const {
        float d = f16_to_f32((uint16_t)(v.h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(v.h.x >> 16));
        float d16 = d * 0.0625f;
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(v.h.y, v.h.z, v.h.w, sc_lo, sc_hi, m_lo, m_hi);
        uint32_t w[8] = {v.q[0].x, v.q[0].y, v.q[1].x, v.q[1].y, v.q[2].x, v.q[2].y, v.q[3].x, v.q[3].y};
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
    static constexpr int XSTEP = 64;
};

template <>
struct Blk<kQ6K> {
    static constexpr int DEPTH = 5;
    struct Data { uint4 la, lb, hh, sv; uint32_t d; };
    const uint4 *lp, *hp, *sp;
    const uint16_t *dp;
    __device__ Blk(const Planes &p, int64_t row, int t)
        : lp(reinterpret_cast<const uint4 *>(p.qs + row * p.nb * 128 + 32 * t)),
          hp(reinterpret_cast<const uint4 *>(p.aux + row * p.nb * 64 + 16 * t)),
          sp(reinterpret_cast<const uint4 *>(p.sc + row * p.nb * 16)), dp(p.d + row * p.nb) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const {
        v.la = lp[8 * b];
        v.lb = lp[8 * b + 1];
        v.hh = hp[4 * b];
        v.sv = sp[b];
        v.d = dp[b];
    }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb, int t) const {
        float d = f16_to_f32((uint16_t)v.d);
        uint32_t scw[4] = {v.sv.x, v.sv.y, v.sv.z, v.sv.w};
        const int th = t >> 1;
#pragma unroll
        for (int n = 0; n < 2; n++) {
            uint32_t A0 = n ? v.lb.x : v.la.x, A1 = n ? v.lb.y : v.la.y;  // ql[64n + 8t + l]
            uint32_t B0 = n ? v.lb.z : v.la.z, B1 = n ? v.lb.w : v.la.w;  // ql[64n + 32 + 8t + l]
            uint32_t H0 = n ? v.hh.z : v.hh.x, H1 = n ? v.hh.w : v.hh.y;  // qh[32n + 8t + l]
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
    static constexpr int XSTEP = 64;
};

template <int DT, bool ACC, int THREADS, int IO = TRHIP_F32>
__global__ __launch_bounds__(THREADS) void gemv_exact_kernel(const Planes p, const void *__restrict__ x,
                                                             void *__restrict__ c, int64_t N, int64_t row0, int64_t K) {
    extern __shared__ float4 xs[];  // K / 4 float4: the whole activation vector
    const int t = threadIdx.x & 3;
    const int64_t r = (int64_t)blockIdx.x * (THREADS / 4) + (threadIdx.x >> 2);
    const bool live = r < N;
    const int64_t row = row0 + (live ? r : 0);
    const int64_t nb = p.nb;
    using B = Blk<DT>;
    constexpr int D = B::DEPTH;
    B blk(p, row, t);
    typename B::Data ring[D];
    // x (cache-resident) and the first weight blocks (from HBM) in flight together, then x into LDS
    XStager<THREADS, IO> xst;
    xst.issue(x, K / 4, 0);
    __builtin_amdgcn_sched_barrier(0);  // x is requested first: the wait before its stores then skips the weights
#pragma unroll
    for (int s = 0; s < D; s++) blk.load(ring[s], s < nb ? s : nb - 1);
    xst.commit(xs, K / 4, 0);
    xst.rest(xs, x, K / 4);
    __syncthreads();

    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; l++) acc[l] = 0.0f;
    const float4 *xl = xs + 2 * t;
    // Loads are unconditional (clamped to the last block, re-reading it at the tail) so the ring stays
    // in registers with static indices. Full passes of the D-block ring run without a branch, so the LDS reads of x for
    // several blocks are issued before their first use; the last nb % D blocks, already in the ring, follow.
    const int64_t nfull = nb - nb % D;
    for (int64_t b0 = 0; b0 < nfull; b0 += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            const int64_t b = b0 + s;
            typename B::Data cur = ring[s];
            blk.load(ring[s], (b + D < nb) ? b + D : nb - 1);
            blk.compute(acc, cur, xl + B::XSTEP * b, t);
        }
    }
#pragma unroll
    for (int s = 0; s < D; s++)
        if (nfull + s < nb) blk.compute(acc, ring[s], xl + B::XSTEP * (nfull + s), t);
    float res = sdot32_tree(acc);
    if (live && t == 0) put_out<ACC, IO>(c, r, res);
}

// ---------------------------------------------------------------- eight lanes per row
// The same arithmetic with twice the lanes per row: lane u (0..7) owns the four chains 4u..4u+3 (half u&1 of
// sdot32 register u>>1), i.e. elements 32G + 4u .. +3 of every 32-element group G in ascending G. Each lane
// reads aligned 4-byte pieces of the same plane layout. The tree: (A0+A1) and (A2+A3) by xor-shuffle 2, their
// sum by xor 4, s_l = Y[l] + Y[l+4] by xor 1, then (s0+s2)+(s1+s3) in-lane; IEEE addition is commutative, so
// the partners of every shuffle hold identical bits.
template <int DT>
struct Blk8;

template <>
struct Blk8<kQ8> {
    static constexpr int DEPTH = 24;
    struct Data { uint32_t q, d; };
    const uint32_t *qp;
    const uint16_t *dp;
    __device__ Blk8(const Planes &p, int64_t row, int u)
        : qp(reinterpret_cast<const uint32_t *>(p.qs + row * p.nb * 32) + u), dp(p.d + row * p.nb) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const { v.q = qp[8 * b]; v.d = dp[b]; }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb) const {
        const float d = f16_to_f32((uint16_t)v.d);
        fma4(acc, v.q ^ 0x80808080u, d, -128.0f * d, xb[0]);  // (u - 128)*d exact
    }
    static constexpr int XSTEP = 8;  // float4s of x per block
};

template <>
struct Blk8<kQ4> {
    static constexpr int DEPTH = 24;
    struct Data { uint32_t q, d; };
    const uint32_t *qp;
    const uint16_t *dp;
    int sh;
    __device__ Blk8(const Planes &p, int64_t row, int u)
        : qp(reinterpret_cast<const uint32_t *>(p.qs + row * p.nb * 16) + (u & 3)), dp(p.d + row * p.nb),
          sh(u >= 4 ? 4 : 0) {}  // lanes 4..7 take the high nibbles (elements 16..31)
    __device__ __forceinline__ void load(Data &v, int64_t b) const { v.q = qp[4 * b]; v.d = dp[b]; }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb) const {
        const float d = f16_to_f32((uint16_t)v.d);
        fma4(acc, (v.q >> sh) & 0x0F0F0F0Fu, d, -8.0f * d, xb[0]);
    }
    static constexpr int XSTEP = 8;
};

template <>
struct Blk8<kQ4K> {
    static constexpr int DEPTH = 6;
    struct Data { uint4 h; uint32_t q[4]; };
    const uint4 *hp;
    const uint32_t *qp;  // lane u's 4 bytes of group pair g: 64(u>>2) + 16g + 8((u>>1)&1) + 4(u&1)
    __device__ Blk8(const Planes &p, int64_t row, int u)
        : hp(reinterpret_cast<const uint4 *>(p.aux + row * p.nb * 16)),
          qp(reinterpret_cast<const uint32_t *>(p.qs + row * p.nb * 128) + 16 * (u >> 2) + 2 * ((u >> 1) & 1) + (u & 1)) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const {
        v.h = hp[b];
#pragma unroll
        for (int g = 0; g < 4; g++) v.q[g] = qp[32 * b + 4 * g];
    }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb) const {
        const float d = f16_to_f32((uint16_t)(v.h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(v.h.x >> 16));
        const float d16 = d * 0.0625f;
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(v.h.y, v.h.z, v.h.w, sc_lo, sc_hi, m_lo, m_hi);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
            const int k0 = (2 * g) & 3, k1 = (2 * g + 1) & 3;
            const float s0 = d * ubyte_f(scw, k0), n0 = -(dmin * ubyte_f(mw, k0));
            const float s1 = d16 * ubyte_f(scw, k1), n1 = -(dmin * ubyte_f(mw, k1));
            // sub-block 2g: low nibbles; sub-block 2g+1: high nibbles read as 16*code with scale d/16 (exact)
            fma4(acc, v.q[g] & 0x0F0F0F0Fu, s0, n0, xb[8 * (2 * g)]);
            fma4(acc, v.q[g] & 0xF0F0F0F0u, s1, n1, xb[8 * (2 * g + 1)]);
        }
    }
    static constexpr int XSTEP = 64;
};

template <>
struct Blk8<kQ6K> {
    static constexpr int DEPTH = 4;
    struct Data { uint32_t l[4], hq[2]; uint4 sv; uint32_t d; };
    const uint32_t *lp, *hp;
    const uint4 *sp;
    const uint16_t *dp;
    int th;
    __device__ Blk8(const Planes &p, int64_t row, int u)
        : lp(reinterpret_cast<const uint32_t *>(p.qs + row * p.nb * 128) + 8 * (u >> 1) + (u & 1)),
          hp(reinterpret_cast<const uint32_t *>(p.aux + row * p.nb * 64) + 4 * (u >> 1) + (u & 1)),
          sp(reinterpret_cast<const uint4 *>(p.sc + row * p.nb * 16)), dp(p.d + row * p.nb), th(u >> 2) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const {
#pragma unroll
        for (int i = 0; i < 4; i++) v.l[i] = lp[32 * b + 2 * i];  // ql bytes 32(u>>1) + 16n + 8h + 4(u&1), i = 2n + h
#pragma unroll
        for (int n = 0; n < 2; n++) v.hq[n] = hp[16 * b + 2 * n];  // qh bytes 16(u>>1) + 8n + 4(u&1)
        v.sv = sp[b];
        v.d = dp[b];
    }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float4 *xb) const {
        const float d = f16_to_f32((uint16_t)v.d);
        const uint32_t scw[4] = {v.sv.x, v.sv.y, v.sv.z, v.sv.w};
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t A = v.l[2 * n + (k & 1)];
                const uint32_t nib = (k < 2) ? (A & 0x0F0F0F0Fu) : ((A >> 4) & 0x0F0F0F0Fu);
                const uint32_t code = nib | (((v.hq[n] >> (2 * k)) & 0x03030303u) << 4);
                const int si = 8 * n + 2 * k + th;  // 16-element scale of elements 4u..4u+3 of group 4n + k
                const int8_t scv = (int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xFF);
                const float ds = d * (float)scv;  // exact (11 x 8 bits)
                // fl(ds*(code-32)) == fmaf(ds, code, -32*ds): same real number, one rounding
                fma4(acc, code, ds, -32.0f * ds, xb[8 * (4 * n + k)]);
            }
    }
    static constexpr int XSTEP = 64;
};

__device__ __forceinline__ float sdot32_tree8(const float *acc) {
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float p = acc[i] + __shfl_xor(acc[i], 2);  // A0+A1 (lanes 0-3), A2+A3 (lanes 4-7)
        const float y = p + __shfl_xor(p, 4);            // Y[4(u&1) + i]
        s[i] = y + __shfl_xor(y, 1);                     // s_i = Y[i] + Y[i+4]
    }
    return (s[0] + s[2]) + (s[1] + s[3]);
}

template <int DT, bool ACC, int THREADS, int IO = TRHIP_F32>
__global__ __launch_bounds__(THREADS) void gemv_exact8_kernel(const Planes p, const void *__restrict__ x,
                                                              void *__restrict__ c, int64_t N, int64_t row0, int64_t K) {
    extern __shared__ float4 xs[];  // K / 4 float4: the whole activation vector
    const int u = threadIdx.x & 7;
    const int64_t r = (int64_t)blockIdx.x * (THREADS / 8) + (threadIdx.x >> 3);
    const bool live = r < N;
    const int64_t row = row0 + (live ? r : 0);
    const int64_t nb = p.nb;
    using B = Blk8<DT>;
    constexpr int D = B::DEPTH;
    B blk(p, row, u);
    typename B::Data ring[D];
    XStager<THREADS, IO> xst;
    xst.issue(x, K / 4, 0);
    __builtin_amdgcn_sched_barrier(0);  // x is requested first: the wait before its stores then skips the weights
#pragma unroll
    for (int s = 0; s < D; s++) blk.load(ring[s], s < nb ? s : nb - 1);
    xst.commit(xs, K / 4, 0);
    xst.rest(xs, x, K / 4);
    __syncthreads();

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const float4 *xl = xs + u;
    // full passes of the D-block ring without a branch, then the last nb % D blocks from the ring (as in the four-lane
    // kernel)
    const int64_t nfull = nb - nb % D;
    for (int64_t b0 = 0; b0 < nfull; b0 += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            const int64_t b = b0 + s;
            typename B::Data cur = ring[s];
            blk.load(ring[s], (b + D < nb) ? b + D : nb - 1);
            blk.compute(acc, cur, xl + B::XSTEP * b);
        }
    }
#pragma unroll
    for (int s = 0; s < D; s++)
        if (nfull + s < nb) blk.compute(acc, ring[s], xl + B::XSTEP * (nfull + s));
    const float res = sdot32_tree8(acc);
    if (live && u == 0) put_out<ACC, IO>(c, r, res);
}

// ---------------------------------------------------------------- sixteen lanes per row
// For stores whose rows alone leave SIMDs idle (4096 rows x 8 lanes is 512 waves for 1024 SIMDs): lane v (0..15)
// owns the two chains 2v, 2v+1 (lanes 2(v&3), 2(v&3)+1 of sdot32 register v>>2), i.e. elements 32G + 2v, 2v+1 of
// every 32-element group G in ascending G. The row's 16 lanes read the block's 16 (q4_0) or 32 (q8_0) code bytes as
// one contiguous piece, two bytes per lane (q4_k: four 2-byte pieces per block, one per group pair; q6_k: the
// eight-lane pieces split in two). The tree: A0+A1 and A2+A3 by xor-shuffle 4, their sum (Y) by xor 8,
// s_l = Y[l] + Y[l+4] by xor 2, (s0+s2) and (s1+s3) by xor 1, their sum in-lane; IEEE addition is commutative,
// so the partners of every shuffle hold identical bits.
// VOL: hide the codes with a volatile statement, which also keeps the loads in program order around it (faster for
// the q8_0 / q4_0 blocks, two elements per lane: 4096x14336 30.4 against 32.2 us)
template <bool VOL>
__device__ __forceinline__ void fma2(float *acc, uint32_t codes, float s, float negm, float2 xv) {
    codes = VOL ? opaque(codes) : hide(codes);
    acc[0] = fmaf(fmaf(s, ubyte_f(codes, 0), negm), xv.x, acc[0]);
    acc[1] = fmaf(fmaf(s, ubyte_f(codes, 1), negm), xv.y, acc[1]);
}

template <int DT>
struct Blk16;

template <>
struct Blk16<kQ8> {
    static constexpr int DEPTH = 24;
    struct Data { uint32_t q, d; };
    const uint16_t *qp;
    const uint16_t *dp;
    __device__ Blk16(const Planes &p, int64_t row, int v)
        : qp(reinterpret_cast<const uint16_t *>(p.qs + row * p.nb * 32) + v), dp(p.d + row * p.nb) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const { v.q = qp[16 * b]; v.d = dp[b]; }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float2 *xb) const {
        const float d = f16_to_f32((uint16_t)v.d);
        fma2<true>(acc, v.q ^ 0x8080u, d, -128.0f * d, xb[0]);  // (u - 128)*d exact
    }
    static constexpr int XSTEP = 16;  // float2s of x per block
};

template <>
struct Blk16<kQ4> {
    static constexpr int DEPTH = 24;
    struct Data { uint32_t q, d; };
    const uint16_t *qp;
    const uint16_t *dp;
    int sh;
    __device__ Blk16(const Planes &p, int64_t row, int v)
        : qp(reinterpret_cast<const uint16_t *>(p.qs + row * p.nb * 16) + (v & 7)), dp(p.d + row * p.nb),
          sh(v >= 8 ? 4 : 0) {}  // lanes 8..15 take the high nibbles (elements 16..31)
    __device__ __forceinline__ void load(Data &v, int64_t b) const { v.q = qp[8 * b]; v.d = dp[b]; }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float2 *xb) const {
        const float d = f16_to_f32((uint16_t)v.d);
        fma2<true>(acc, (v.q >> sh) & 0x0F0Fu, d, -8.0f * d, xb[0]);
    }
    static constexpr int XSTEP = 16;
};

template <>
struct Blk16<kQ4K> {
    static constexpr int DEPTH = 6;
    struct Data { uint4 h; uint32_t q[4]; };
    const uint4 *hp;
    // lane v's two code bytes of group pair g (elements 2v, 2v+1 of sub-blocks 2g and 2g+1) in the lane-sliced qs
    // plane: byte 64((v>>2)>>1) + 16g + 8((v>>2)&1) + 2(v&3)
    const uint16_t *qp;
    __device__ Blk16(const Planes &p, int64_t row, int v)
        : hp(reinterpret_cast<const uint4 *>(p.aux + row * p.nb * 16)),
          qp(reinterpret_cast<const uint16_t *>(p.qs + row * p.nb * 128) + 32 * (v >> 3) + 4 * ((v >> 2) & 1) + (v & 3)) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const {
        v.h = hp[b];
#pragma unroll
        for (int g = 0; g < 4; g++) v.q[g] = qp[64 * b + 8 * g];
    }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float2 *xb) const {
        const float d = f16_to_f32((uint16_t)(v.h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(v.h.x >> 16));
        const float d16 = d * 0.0625f;
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(v.h.y, v.h.z, v.h.w, sc_lo, sc_hi, m_lo, m_hi);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
            const int k0 = (2 * g) & 3, k1 = (2 * g + 1) & 3;
            const float s0 = d * ubyte_f(scw, k0), n0 = -(dmin * ubyte_f(mw, k0));
            const float s1 = d16 * ubyte_f(scw, k1), n1 = -(dmin * ubyte_f(mw, k1));
            // sub-block 2g: low nibbles; sub-block 2g+1: high nibbles read as 16*code with scale d/16 (exact)
            fma2<false>(acc, v.q[g] & 0x0F0Fu, s0, n0, xb[16 * (2 * g)]);
            fma2<false>(acc, v.q[g] & 0xF0F0u, s1, n1, xb[16 * (2 * g + 1)]);
        }
    }
    static constexpr int XSTEP = 128;
};

template <>
struct Blk16<kQ6K> {
    static constexpr int DEPTH = 4;
    struct Data { uint32_t l[4], hq[2]; uint4 sv; uint32_t d; };
    // lane v's elements 2v, 2v+1 sit in the two bytes at 2(v&1) of the eight-lane kernel's 4-byte pieces of lane
    // v>>1: ql bytes 32(v>>2) + 4((v>>1)&1) + 2(v&1) + 16n + 8h, qh bytes 16(v>>2) + 4((v>>1)&1) + 2(v&1) + 8n
    const uint16_t *lp, *hp;
    const uint4 *sp;
    const uint16_t *dp;
    int th;
    __device__ Blk16(const Planes &p, int64_t row, int v)
        : lp(reinterpret_cast<const uint16_t *>(p.qs + row * p.nb * 128) + 16 * (v >> 2) + 2 * ((v >> 1) & 1) + (v & 1)),
          hp(reinterpret_cast<const uint16_t *>(p.aux + row * p.nb * 64) + 8 * (v >> 2) + 2 * ((v >> 1) & 1) + (v & 1)),
          sp(reinterpret_cast<const uint4 *>(p.sc + row * p.nb * 16)), dp(p.d + row * p.nb), th(v >> 3) {}
    __device__ __forceinline__ void load(Data &v, int64_t b) const {
#pragma unroll
        for (int i = 0; i < 4; i++) v.l[i] = lp[64 * b + 4 * i];  // i = 2n + h
#pragma unroll
        for (int n = 0; n < 2; n++) v.hq[n] = hp[32 * b + 4 * n];
        v.sv = sp[b];
        v.d = dp[b];
    }
    __device__ __forceinline__ void compute(float *acc, const Data &v, const float2 *xb) const {
        const float d = f16_to_f32((uint16_t)v.d);
        const uint32_t scw[4] = {v.sv.x, v.sv.y, v.sv.z, v.sv.w};
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t A = v.l[2 * n + (k & 1)];
                const uint32_t nib = (k < 2) ? (A & 0x0F0Fu) : ((A >> 4) & 0x0F0Fu);
                const uint32_t code = nib | (((v.hq[n] >> (2 * k)) & 0x0303u) << 4);
                const int si = 8 * n + 2 * k + th;  // 16-element scale of elements 2v, 2v+1 of group 4n + k
                const int8_t scv = (int8_t)((scw[si >> 2] >> (8 * (si & 3))) & 0xFF);
                const float ds = d * (float)scv;  // exact (11 x 8 bits)
                // fl(ds*(code-32)) == fmaf(ds, code, -32*ds): same real number, one rounding
                fma2<false>(acc, code, ds, -32.0f * ds, xb[16 * (4 * n + k)]);
            }
    }
    static constexpr int XSTEP = 128;
};

__device__ __forceinline__ float sdot32_tree16(const float *acc) {
    float e[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const float a = acc[i] + __shfl_xor(acc[i], 4);  // A0+A1 (lanes 0-7), A2+A3 (lanes 8-15) at l = 2(v&3) + i
        const float y = a + __shfl_xor(a, 8);            // Y[2(v&3) + i]
        const float sl = y + __shfl_xor(y, 2);           // s_i (v&3 = 0, 2) or s_{2+i} (v&3 = 1, 3)
        e[i] = sl + __shfl_xor(sl, 1);                   // s_i + s_{2+i}
    }
    return e[0] + e[1];  // (s0+s2) + (s1+s3)
}

template <int DT, bool ACC, int THREADS, int IO>
__device__ __forceinline__ void exact16_body(const Planes p, const void *__restrict__ x, void *__restrict__ c, int64_t N,
                                             int64_t row0, int64_t K) {
    extern __shared__ float4 xs[];  // K / 4 float4: the whole activation vector
    const int v = threadIdx.x & 15;
    const int64_t r = (int64_t)blockIdx.x * (THREADS / 16) + (threadIdx.x >> 4);
    const bool live = r < N;
    const int64_t row = row0 + (live ? r : 0);
    const int64_t nb = p.nb;
    using B = Blk16<DT>;
    constexpr int D = B::DEPTH;
    B blk(p, row, v);
    typename B::Data ring[D];
    XStager<THREADS, IO> xst;
    xst.issue(x, K / 4, 0);
    __builtin_amdgcn_sched_barrier(0);  // x is requested first: the wait before its stores then skips the weights
#pragma unroll
    for (int s = 0; s < D; s++) blk.load(ring[s], s < nb ? s : nb - 1);
    xst.commit(xs, K / 4, 0);
    xst.rest(xs, x, K / 4);
    __syncthreads();

    float acc[2] = {0.0f, 0.0f};
    const float2 *xl = reinterpret_cast<const float2 *>(xs) + v;
    // full passes of the D-block ring without a branch, then the last nb % D blocks from the ring (as in the four-lane
    // kernel)
    const int64_t nfull = nb - nb % D;
    for (int64_t b0 = 0; b0 < nfull; b0 += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            const int64_t b = b0 + s;
            typename B::Data cur = ring[s];
            blk.load(ring[s], (b + D < nb) ? b + D : nb - 1);
            blk.compute(acc, cur, xl + B::XSTEP * b);
        }
    }
#pragma unroll
    for (int s = 0; s < D; s++)
        if (nfull + s < nb) blk.compute(acc, ring[s], xl + B::XSTEP * (nfull + s));
    const float res = sdot32_tree16(acc);
    if (live && v == 0) put_out<ACC, IO>(c, r, res);
}

template <int DT, bool ACC, int THREADS, int IO = TRHIP_F32>
__global__ __launch_bounds__(THREADS) void gemv_exact16_kernel(const Planes p, const void *__restrict__ x,
                                                               void *__restrict__ c, int64_t N, int64_t row0, int64_t K) {
    exact16_body<DT, ACC, THREADS, IO>(p, x, c, N, row0, K);
}

// The same with the register budget of one wave per SIMD, for grids of at most one wave per SIMD: the compiler then
// issues a block's LDS reads of x ahead of their use instead of waiting for each (q4_k 4096x14336 26.3 -> 22.2 us,
// 4096x4096 9.45 -> 8.39; q6_k 4096x14336 28.6 -> 24.6).
template <int DT, bool ACC, int THREADS, int IO = TRHIP_F32>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemv_exact16w1_kernel(
    const Planes p, const void *__restrict__ x, void *__restrict__ c, int64_t N, int64_t row0, int64_t K) {
    exact16_body<DT, ACC, THREADS, IO>(p, x, c, N, row0, K);
}

template <int DT, int THREADS, int MINW>
void launch_exact16_t(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                      bool acc, size_t lds, int io) {
    dim3 grid((unsigned)((N + THREADS / 16 - 1) / (THREADS / 16))), block(THREADS);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, lds, ctx->stream, w->planes(), x, c, N, row0, w->K); };
    if constexpr (MINW == 1) {
        if (io == TRHIP_F16) acc ? go(gemv_exact16w1_kernel<DT, true, THREADS, TRHIP_F16>) : go(gemv_exact16w1_kernel<DT, false, THREADS, TRHIP_F16>);
        else if (io == TRHIP_BF16) acc ? go(gemv_exact16w1_kernel<DT, true, THREADS, TRHIP_BF16>) : go(gemv_exact16w1_kernel<DT, false, THREADS, TRHIP_BF16>);
        else acc ? go(gemv_exact16w1_kernel<DT, true, THREADS>) : go(gemv_exact16w1_kernel<DT, false, THREADS>);
    } else {
        if (io == TRHIP_F16) acc ? go(gemv_exact16_kernel<DT, true, THREADS, TRHIP_F16>) : go(gemv_exact16_kernel<DT, false, THREADS, TRHIP_F16>);
        else if (io == TRHIP_BF16) acc ? go(gemv_exact16_kernel<DT, true, THREADS, TRHIP_BF16>) : go(gemv_exact16_kernel<DT, false, THREADS, TRHIP_BF16>);
        else acc ? go(gemv_exact16_kernel<DT, true, THREADS>) : go(gemv_exact16_kernel<DT, false, THREADS>);
    }
}

template <int DT, int THREADS>
void launch_exact8_t(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                     bool acc, size_t lds, int io) {
    dim3 grid((unsigned)((N + THREADS / 8 - 1) / (THREADS / 8))), block(THREADS);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, lds, ctx->stream, w->planes(), x, c, N, row0, w->K); };
    if (io == TRHIP_F16) acc ? go(gemv_exact8_kernel<DT, true, THREADS, TRHIP_F16>) : go(gemv_exact8_kernel<DT, false, THREADS, TRHIP_F16>);
    else if (io == TRHIP_BF16) acc ? go(gemv_exact8_kernel<DT, true, THREADS, TRHIP_BF16>) : go(gemv_exact8_kernel<DT, false, THREADS, TRHIP_BF16>);
    else acc ? go(gemv_exact8_kernel<DT, true, THREADS>) : go(gemv_exact8_kernel<DT, false, THREADS>);
}

template <int DT, int THREADS>
void launch_exact_t(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                    bool acc, size_t lds, int io) {
    dim3 grid((unsigned)((N + THREADS / 4 - 1) / (THREADS / 4))), block(THREADS);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, lds, ctx->stream, w->planes(), x, c, N, row0, w->K); };
    if (io == TRHIP_F16) acc ? go(gemv_exact_kernel<DT, true, THREADS, TRHIP_F16>) : go(gemv_exact_kernel<DT, false, THREADS, TRHIP_F16>);
    else if (io == TRHIP_BF16) acc ? go(gemv_exact_kernel<DT, true, THREADS, TRHIP_BF16>) : go(gemv_exact_kernel<DT, false, THREADS, TRHIP_BF16>);
    else acc ? go(gemv_exact_kernel<DT, true, THREADS>) : go(gemv_exact_kernel<DT, false, THREADS>);
}

// Rows per workgroup: the largest of 64, 32, 16 that still gives >= 200 workgroups (64 measured fastest on
// 14336 rows); trhip_set_launch_shape(TRHIP_KNOB_EXACT_ROWS) overrides.
int gemv_rows_per_wg(const trhip_ctx *ctx, int64_t N) {
    if (ctx->force_exact_rows) return ctx->force_exact_rows;
    if (N >= 64 * 200) return 64;
    if (N >= 32 * 200) return 32;
    return 16;
}

template <int DT>
int launch_exact(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                 bool acc, int io = TRHIP_F32) {
    size_t lds = (size_t)w->K * sizeof(float);
    if (lds > 160 * 1024) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemv: K too large for the LDS copy of x");
    // lanes per row: 8 measured faster for q4_k (14336x4096 cold: 15.7 vs 18.0 us; 1024x4096: 12.5 vs 15.9),
    // q8_0 (4096x4096: 20.3 vs 23.6) and equal for q4_0; for q6_k 4 stays faster on large grids (14336x4096: 17.8 vs
    // 19.9 us, 128256x4096: 109 vs 139) and 8 wins below 10240 rows (1024x4096 15.0 -> 10.9, 4096x4096 15.5 -> 11.2,
    // 4096x14336 47.7 -> 34.5; bit-identical). trhip_set_launch_shape(TRHIP_KNOB_EXACT_LANES) overrides.
    // 16 lanes up to 48 rows per CU (12288 on 256 CUs: at most three 16-row workgroups per CU), where 8 leave SIMDs
    // idle or 16 still balance (cold, us, 8 -> 16 lanes, bit-identical: q4_k 4096x14336 32.9 -> 26.3, 4096x4096
    // 11.0 -> 9.4, 12288x4096 13.2 -> 12.9; q6_k 4096x14336 34.9 -> 28.6, 10240x4096 19.3 -> 14.6; q4_0 4096x14336
    // 41.3 -> 30.4; q8_0 4096x4096 15.0 -> 12.0). Above that a fourth workgroup lands on some CUs and 16 lanes lose
    // (q4_k 13312x4096 13.7 -> 15.5, 14336x4096 14.1 -> 15.9), except q8_0 from 80 rows per CU (20480x4096 32.3 ->
    // 29.4, 28672x4096 48.7 -> 37.5). q6_k keeps 4 lanes on large grids (128256x4096: 117 against 130 on 16).
    const int64_t cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    const int lanes = ctx->force_exact_lanes ? ctx->force_exact_lanes
                      : (N <= 48 * cus || (DT == kQ8 && N >= 80 * cus)) ? 16
                      : (DT == kQ6K ? 4 : 8);
    if (lanes == 16) {
        // rows per workgroup: the most (16, 8, 4) that still give 256 workgroups; the k-quants take the one-wave
        // register budget up to 4096 rows (at most 1024 waves; 6144x4096 measured 10.8 -> 15.1 us with it), q8_0 and
        // q4_0 never (4096x14336: 30.4 -> 32.4 us)
        constexpr bool kq = DT == kQ4K || DT == kQ6K;
        if (N > 4096 || !kq) {
            if (N >= 16 * 256) launch_exact16_t<DT, 256, 4>(ctx, w, row0, N, x, c, acc, lds, io);
            else if (N >= 8 * 256) launch_exact16_t<DT, 128, 4>(ctx, w, row0, N, x, c, acc, lds, io);
            else launch_exact16_t<DT, 64, 4>(ctx, w, row0, N, x, c, acc, lds, io);
        } else if (N >= 16 * 256) launch_exact16_t<DT, 256, 1>(ctx, w, row0, N, x, c, acc, lds, io);
        else if (N >= 8 * 256) launch_exact16_t<DT, 128, 1>(ctx, w, row0, N, x, c, acc, lds, io);
        else launch_exact16_t<DT, 64, 1>(ctx, w, row0, N, x, c, acc, lds, io);
        return launch_check(ctx, "gemv_exact16");
    }
    if (lanes >= 8) {
        // 8 lanes per row: 32 rows per 256-thread workgroup, 16 per 128-thread one and 8 per 64-thread one as N falls
        // (cold, us, 128 -> 64 threads, bit-identical: q4_k 1024x4096 11.0 -> 10.66, 2048x4096 11.1 -> 10.8,
        // 1024x14336 33.6 -> 32.1; q8_0 / q4_0 1024x4096 18.3 / 18.1 -> 17.9 / 17.2); q4_k keeps 16 rows per workgroup
        // on large grids too (14336x4096 13.86 -> 13.7, 28672x4096 22.8 -> 22.4; q8_0 / q4_0 lose 1%)
        if (N >= 32 * 200 && DT != kQ4K) launch_exact8_t<DT, 256>(ctx, w, row0, N, x, c, acc, lds, io);
        else if (N >= 16 * 200) launch_exact8_t<DT, 128>(ctx, w, row0, N, x, c, acc, lds, io);
        else launch_exact8_t<DT, 64>(ctx, w, row0, N, x, c, acc, lds, io);
        return launch_check(ctx, "gemv_exact8");
    }
    switch (gemv_rows_per_wg(ctx, N)) {
    case 64: launch_exact_t<DT, 256>(ctx, w, row0, N, x, c, acc, lds, io); break;
    case 32: launch_exact_t<DT, 128>(ctx, w, row0, N, x, c, acc, lds, io); break;
    default: launch_exact_t<DT, 64>(ctx, w, row0, N, x, c, acc, lds, io); break;
    }
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

// The exact GEMV with f16 / bf16 x (8-byte aligned) and c of that type: x widened on its way into LDS, c widened,
// the row's result added, rounded once (the bits of the fp32 call on the widened values, rounded).
int launch_gemv_exact_io(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                         bool acc, int io) {
    if (N == 0) return TRHIP_OK;
    switch (w->dtype) {
    case kQ8: return launch_exact<kQ8>(ctx, w, row0, N, x, c, acc, io);
    case kQ4: return launch_exact<kQ4>(ctx, w, row0, N, x, c, acc, io);
    case kQ4K: return launch_exact<kQ4K>(ctx, w, row0, N, x, c, acc, io);
    case kQ6K: return launch_exact<kQ6K>(ctx, w, row0, N, x, c, acc, io);
    }
    return fail(ctx, TRHIP_ERR_INVALID, "gemv: bad dtype");
}

}  // namespace trhip
