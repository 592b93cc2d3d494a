// gemm_rows.hip -- fp32-activation quant matmul for M > 1, bit-identical to TR's CPU order.
//
// tensor/cpu_quant.go:103-147 (quantGemmPanels) and the tile path (:59-82, gemmPart in
// cpu_matmul.go:330-380) both compute, for every output (m, n): for each 256-deep K chunk a fresh
// fused chain from +0 in ascending k (sgemm6x16, cpu_micro_amd64.s:14-64), the chunk results added
// in chunk order into a cleared `part`, then c[m, n] += part.
//
// Mapping: a wave is 64 weight rows (lane = row) on one 256-deep chunk; it decodes its rows' weights 32
// elements at a time, exactly as tensor/quant.go does, and advances MB activation rows' chains together, so
// every decoded weight feeds MB fused multiply-adds. The activations of a 32-element group are the same for all
// lanes: the wave stages them from a k-major copy xt[k][m] into its own LDS slice and reads them back as
// broadcasts; weights and activations of the next group are requested before the current group's arithmetic.
// A workgroup is 16 such
// waves on 16 consecutive chunks of the same 64 rows; their chain results meet in LDS, and 1024 threads
// (one per (m, row)) add them to `part` in chunk order, 16 chunks at a time.
#include "trhip_internal.hpp"

namespace trhip {
namespace {

constexpr int kWaves = 16;  // chunk-waves per workgroup
constexpr int kMaxMB = 16;

// 32 consecutive elements (group G of a 32-element grid along the row) of block bi, exactly as
// tensor/quant.go:139-205: load() fetches the bytes (issued one group ahead), decode() turns them into floats.
template <int DT>
struct Group;

template <>
struct Group<kQ8> {
    uint4 a, b;
    uint32_t d;
    __device__ __forceinline__ void load(const Planes p, int64_t bi, int) {
        const uint4 *q = reinterpret_cast<const uint4 *>(p.qs + bi * 32);
        a = q[0];
        b = q[1];
        d = p.d[bi];
    }
    __device__ __forceinline__ void decode(int, float y[32]) const {
        const float dv = f16_to_f32((uint16_t)d), nd = -128.0f * dv;  // q*d = d*(u - 128), u = q + 128: exact
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t u = opaque(w[i] ^ 0x80808080u);
#pragma unroll
            for (int k = 0; k < 4; k++) y[4 * i + k] = fmaf(dv, ubyte_f(u, k), nd);
        }
    }
};

template <>
struct Group<kQ4> {
    uint4 a;
    uint32_t d;
    __device__ __forceinline__ void load(const Planes p, int64_t bi, int) {
        a = *reinterpret_cast<const uint4 *>(p.qs + bi * 16);
        d = p.d[bi];
    }
    __device__ __forceinline__ void decode(int, float y[32]) const {
        const float dv = f16_to_f32((uint16_t)d), n8 = -8.0f * dv;  // (q - 8)*d, exact
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = opaque(w[i] & 0x0F0F0F0Fu), hi = opaque((w[i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                y[4 * i + k] = fmaf(dv, ubyte_f(lo, k), n8);
                y[16 + 4 * i + k] = fmaf(dv, ubyte_f(hi, k), n8);
            }
        }
    }
};

template <>
struct Group<kQ4K> {
    uint4 h, a, b;
    __device__ __forceinline__ void load(const Planes p, int64_t bi, int j) {
        h = *reinterpret_cast<const uint4 *>(p.aux + bi * 16);
        // old bytes 32(j/2) + e sit at 16(j/2) + e (e < 16) and 64 + 16(j/2) + e - 16 of the lane-sliced block
        const uint8_t *qb = p.qs + bi * 128 + 16 * (j >> 1);
        a = *reinterpret_cast<const uint4 *>(qb);
        b = *reinterpret_cast<const uint4 *>(qb + 64);
    }
    __device__ __forceinline__ void decode(int j, float y[32]) const {
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(h.y, h.z, h.w, sc_lo, sc_hi, m_lo, m_hi);
        const int sh = 8 * (j & 3);
        const float d = f16_to_f32((uint16_t)(h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(h.x >> 16));
        const float d1 = d * (float)(((j < 4 ? sc_lo : sc_hi) >> sh) & 0xFF);
        const float m1 = dmin * (float)(((j < 4 ? m_lo : m_hi) >> sh) & 0xFF);
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t nib = opaque((j & 1) ? (w[i] >> 4) & 0x0F0F0F0Fu : w[i] & 0x0F0F0F0Fu);
#pragma unroll
            for (int k = 0; k < 4; k++) y[4 * i + k] = fmaf(d1, ubyte_f(nib, k), -m1);  // d1*q exact: one rounding
        }
    }
};

template <>
struct Group<kQ6K> {
    uint2 ql[4], qh[4];
    uint32_t d, sc;  // sc: the two int8 scales of the group's halves
    __device__ __forceinline__ void load(const Planes p, int64_t bi, int G) {
        const int n = G >> 2, k4 = G & 3;
        const uint8_t *l = p.qs + bi * 128 + 16 * n + 8 * (k4 & 1), *hp = p.aux + bi * 64 + 8 * n;
#pragma unroll
        for (int t = 0; t < 4; t++) {  // elements 8t .. 8t+7
            ql[t] = *reinterpret_cast<const uint2 *>(l + 32 * t);
            qh[t] = *reinterpret_cast<const uint2 *>(hp + 16 * t);
        }
        d = p.d[bi];
        sc = *reinterpret_cast<const uint16_t *>(p.sc + bi * 16 + 8 * n + 2 * k4);
    }
    __device__ __forceinline__ void decode(int G, float y[32]) const {
        const int k4 = G & 3;
        const float dv = f16_to_f32((uint16_t)d);
        const float s0 = dv * (float)(int8_t)(sc & 0xFF), s1 = dv * (float)(int8_t)(sc >> 8);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t lw[2] = {ql[t].x, ql[t].y}, hw[2] = {qh[t].x, qh[t].y};
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const uint32_t nib = (k4 < 2) ? (lw[hh] & 0x0F0F0F0Fu) : ((lw[hh] >> 4) & 0x0F0F0F0Fu);
                const uint32_t code = opaque(nib | (((hw[hh] >> (2 * k4)) & 0x03030303u) << 4));
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int e = 8 * t + 4 * hh + k;
                    y[e] = (e < 16 ? s0 : s1) * (ubyte_f(code, k) - 32.0f);  // fl(fl(d*sc) * (q - 32))
                }
            }
        }
    }
};

// Activations of one 32-element group for MB rows, x[kg + e][m0 + m] (e < 32, m < MB), MB/2 floats per lane.
template <int MB>
struct XGroup {
    float v[MB / 2];
    __device__ __forceinline__ void load(const float *__restrict__ xt, int64_t kg, int64_t M, int64_t m0, int lane) {
#pragma unroll
        for (int u = 0; u < MB / 2; u++) {
            const int i = lane * (MB / 2) + u, e = i / MB, m = i % MB;
            v[u] = xt[(kg + e) * M + m0 + m];
        }
    }
    __device__ __forceinline__ void store(float *xs, int lane) const {
#pragma unroll
        for (int u = 0; u < MB / 2; u++) xs[lane * (MB / 2) + u] = v[u];
    }
};

template <int DT, int MB, bool ACC>
__global__ __launch_bounds__(64 * kWaves) void gemm_rows_kernel(const Planes p, const float *__restrict__ xt,
                                                                float *__restrict__ c, int64_t N, int64_t row0,
                                                                int64_t M, int64_t K, int64_t ldc) {
    __shared__ float part_lds[kWaves][MB][64];
    __shared__ __align__(16) float x_lds[kWaves][32 * MB];  // each wave's activations of its current group
    constexpr int be = block_elems(DT);
    const int lane = threadIdx.x & 63;
    const int cw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t r = (int64_t)blockIdx.x * 64 + lane;
    const int64_t row = row0 + (r < N ? r : N - 1);
    const int64_t nchunks = (K + 255) / 256;
    const int tm = threadIdx.x >> 6;  // summing role: activation row tm of the pass, weight row `lane`
    float *xs = x_lds[cw];
    for (int64_t m0 = 0; m0 < M; m0 += MB) {
        const int64_t mb = (M - m0) < MB ? (M - m0) : MB;
        float part = 0.0f;
        for (int64_t g0 = 0; g0 < nchunks; g0 += kWaves) {
            const int64_t pc = g0 + cw;
            if (pc < nchunks) {  // wave-uniform
                float chain[MB];
#pragma unroll
                for (int m = 0; m < MB; m++) chain[m] = 0.0f;
                const int64_t k0 = pc * 256;
                const int ngroups = (int)(((K - k0) < 256 ? (K - k0) : 256) / 32);
                Group<DT> wg;
                XGroup<MB> xg;
                wg.load(p, row * p.nb + k0 / be, (int)((k0 % be) / 32));
                xg.load(xt, k0, M, m0, lane);
                for (int gi = 0; gi < ngroups; gi++) {
                    const int64_t kg = k0 + 32 * gi;
                    const Group<DT> cur = wg;
                    xg.store(xs, lane);  // the wave's own slice: ordered by the wave's own LDS queue
                    if (gi + 1 < ngroups) {  // next group's bytes are in flight during this group's arithmetic
                        const int64_t kn = kg + 32;
                        wg.load(p, row * p.nb + kn / be, (int)((kn % be) / 32));
                        xg.load(xt, kn, M, m0, lane);
                    }
                    float y[32];
                    cur.decode((int)((kg % be) / 32), y);
                    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's x slice is in LDS
#pragma unroll
                    for (int e = 0; e < 32; e++) {
#pragma unroll
                        for (int q = 0; q < MB / 4; q++) {
                            const float4 xv = *reinterpret_cast<const float4 *>(xs + e * MB + 4 * q);  // broadcast
                            chain[4 * q + 0] = fmaf(xv.x, y[e], chain[4 * q + 0]);
                            chain[4 * q + 1] = fmaf(xv.y, y[e], chain[4 * q + 1]);
                            chain[4 * q + 2] = fmaf(xv.z, y[e], chain[4 * q + 2]);
                            chain[4 * q + 3] = fmaf(xv.w, y[e], chain[4 * q + 3]);
                        }
                    }
                    __builtin_amdgcn_wave_barrier();  // all lanes have read the slice before it is overwritten
                }
#pragma unroll
                for (int m = 0; m < MB; m++) part_lds[cw][m][lane] = chain[m];
            }
            __syncthreads();
            const int ng = (int)((nchunks - g0) < kWaves ? (nchunks - g0) : kWaves);
            if (tm < MB)
                for (int i = 0; i < ng; i++) part = part + part_lds[i][tm][lane];
            __syncthreads();
        }
        if (tm < mb && r < N) {
            float *o = c + (m0 + tm) * ldc + r;
            *o = ACC ? *o + part : part;
        }
    }
}

__global__ void transpose_kernel(const float *__restrict__ x, float *__restrict__ xt, int64_t M, int64_t K) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M * K) return;
    int64_t m = i / K, k = i % K;
    xt[k * M + m] = x[i];
}

template <int DT, int MB>
int run_rows(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *xt, float *c, int64_t M,
             bool acc) {
    dim3 grid((unsigned)((N + 63) / 64)), block(64 * kWaves);
    if (acc)
        hipLaunchKernelGGL((gemm_rows_kernel<DT, MB, true>), grid, block, 0, ctx->stream, w->planes(), xt, c, N, row0, M,
                           w->K, N);
    else
        hipLaunchKernelGGL((gemm_rows_kernel<DT, MB, false>), grid, block, 0, ctx->stream, w->planes(), xt, c, N, row0, M,
                           w->K, N);
    return launch_check(ctx, "gemm_rows");
}

template <int DT>
int run_dt(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *xt, float *c, int64_t M,
           bool acc) {
    if (M >= 16) return run_rows<DT, 16>(ctx, w, row0, N, xt, c, M, acc);
    if (M > 4) return run_rows<DT, 8>(ctx, w, row0, N, xt, c, M, acc);
    return run_rows<DT, 4>(ctx, w, row0, N, xt, c, M, acc);
}

}  // namespace

int launch_gemm_rows(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     int64_t M, bool acc) {
    if (N == 0 || M == 0) return TRHIP_OK;
    int st = TRHIP_OK;
    // the last pass may read up to kMaxMB activations past row M - 1 of the k-major copy: padded, never used
    float *xt = static_cast<float *>(workspace(ctx, (size_t)(M * w->K + kMaxMB) * sizeof(float), &st));
    if (!xt) return st;
    int64_t total = M * w->K;
    hipLaunchKernelGGL(transpose_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, ctx->stream, x, xt, M,
                       w->K);
    if ((st = launch_check(ctx, "transpose")) != TRHIP_OK) return st;
    switch (w->dtype) {
    case kQ8: return run_dt<kQ8>(ctx, w, row0, N, xt, c, M, acc);
    case kQ4: return run_dt<kQ4>(ctx, w, row0, N, xt, c, M, acc);
    case kQ4K: return run_dt<kQ4K>(ctx, w, row0, N, xt, c, M, acc);
    case kQ6K: return run_dt<kQ6K>(ctx, w, row0, N, xt, c, M, acc);
    }
    return fail(ctx, TRHIP_ERR_INVALID, "gemm_rows: bad dtype");
}

}  // namespace trhip
