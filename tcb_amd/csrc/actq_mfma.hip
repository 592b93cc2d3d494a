// actq_mfma.hip -- prefill GEMM with Q8 activations on int8 MFMA (gfx950 v_mfma_i32_32x32x32_i8),
// bit-identical to tensor/cpu_quant_q8.go:91-116 (dotQ4KQ8Go) for q4_k weights.
//
// Per block b and output (m, n) the reference needs two exact integers:
//   isum = sum_j sc_j * sum_{i in j} q4_i * q8_i     msum = sum_j m_j * (bs_2j + bs_2j+1)
// With sc_j = 8*s1 + s0 (s0, s1 < 8) every s*q4 is <= 105, so
//   isum = sum_i (s0 q4)_i q8_i + 8 * sum_i (s1 q4)_i q8_i ,   msum = sum_i m_j(i) q8_i
// are three int8 x int8 dot products over the block's 256 elements: three MFMA accumulations, exact in
// int32. The fp32 epilogue then follows the reference order per block:
//   t = fl(fl(d * fl(isum)) - fl(dmin * fl(msum)));  acc = fl(acc + fl(t * d8))
// with blocks taken in order, so every output is bit-identical to the CPU's single-row kernel.
//
// Tiling: a workgroup (4 waves) computes 64 (m) x 128 (n); wave w owns weight columns 32w .. 32w+31 and all 64
// rows (two 32-row MFMA tiles). Each wave loads its 32 weight rows' q4_k blocks straight into registers and expands
// them there into its B operands (the lane that needs 16 elements of a sub-block holds exactly the 16 code bytes
// they come from), so weights never pass through LDS and every weight byte is expanded once per workgroup. The
// activation codes and the msum operand of a block are staged in LDS (double-buffered, MFMA lane order, one
// barrier per block); the next block's staging loads are in flight while the current block's MFMAs run.
// The 32x32x32 i8 and 32x32x16 f16 operand layouts (lane l: row l%32, k-slice l/32; result reg v: row
// 8(v/4)+4(l/32)+v%4, column l%32) were checked on the device against host matrix products.
#include "trhip_internal.hpp"

#include <cstdlib>

namespace trhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

constexpr int TN = 128, THREADS = 256;
// Per row-tile height TM (64 or 32): LDS staging of one block, in MFMA lane order.
template <int TM>
struct Tile {
    static constexpr int MT = TM / 32;           // 32-row MFMA tiles per wave
    static constexpr int ABYTES = TM * 256;      // activation codes of one block
    static constexpr int SBYTES = TM * 32;       // f16 msum operand of one block
    static constexpr int STAGE = ABYTES + SBYTES + TM * (int)sizeof(float);
    static constexpr size_t LDS = 2 * STAGE + (TM + 1) * sizeof(int);
    static constexpr int CPW = TM / 16;          // 1 KB activation chunks staged per wave (THREADS = 256)
};

// Four bytes (each < 16) times s (< 8) with one packed 16-bit multiply: the products (< 128) stay in
// their bytes, so nothing carries into the neighbour.
__device__ __forceinline__ uint32_t mul4(uint32_t nib4, uint32_t s) {
    us2 a = __builtin_bit_cast(us2, nib4);
    us2 r = a * (us2){(unsigned short)s, (unsigned short)s};
    return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ v4i mul16(uint4 nib, uint32_t s) {
    return (v4i){(int)mul4(nib.x, s), (int)mul4(nib.y, s), (int)mul4(nib.z, s), (int)mul4(nib.w, s)};
}

__device__ __forceinline__ uint32_t pack_h2(uint32_t a, uint32_t b) {  // two small integers as f16 bits
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)b) << 16);
}

// Workgroup -> tile: workgroups are dealt to the 8 XCDs round-robin, so when the tile count allows, XCD x takes a
// contiguous run of column tiles with all their row tiles next to each other: a weight tile is fetched into that
// XCD's L2 once and reused by every row tile.
__device__ __forceinline__ void tile_of(int64_t wg, int64_t mt, int64_t nt, int64_t &tm, int64_t &tn) {
    const int64_t total = mt * nt;
    int64_t t = wg;
    if (total % 8 == 0) t = (wg & 7) * (total / 8) + (wg >> 3);
    tm = t % mt;
    tn = t / mt;
}

// msum = sum_j S_j m_j with S_j = 64 Sh_j + Sl_j: one f16 MFMA over k = [Sh_0..7 | Sl_0..7] x [64 m_0..7 | m_0..7].
// Every product and partial sum is an integer below 2^24, so the fp32 result is msum exactly.
template <bool ACC, int TM>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(TM == 64 ? 2 : 3, TM == 64 ? 2 : 4))) void actq_mfma_q4k(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const int8_t *__restrict__ q, const float *__restrict__ d8, const uint16_t *__restrict__ sj,
    const uint8_t *__restrict__ bad_blk, float *__restrict__ c) {
    using T = Tile<TM>;
    constexpr int MT = T::MT, ABYTES = T::ABYTES, SBYTES = T::SBYTES, STAGE = T::STAGE, CPW = T::CPW;
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowstate = reinterpret_cast<int *>(lds + 2 * STAGE);  // [TM] 0 ok, 1 NaN/Inf row, 2 outside M
    int *anybad = rowstate + TM;                                // some row of the tile is 1

    const int nb = (int)p.nb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + TM - 1) / TM, (N + TN - 1) / TN, tmi, tni);
    const int64_t n0 = tni * TN, m0 = tmi * TM;
    if (tid == 0) *anybad = 0;
    __syncthreads();

    for (int i = tid; i < TM; i += THREADS) {
        int64_t gm = m0 + i;
        int st = 2;
        if (gm < M) {
            st = 0;
            for (int b = 0; b < nb; b++) st |= bad_blk[gm * nb + b] != 0;
            if (st) *anybad = 1;
        }
        rowstate[i] = st;
    }

    // activation staging: wave w stages chunks c = CPW w .. +CPW-1 (tile c / 8, kc c % 8), lane tid & 63 of each;
    // threads < 2 TM also stage the msum operand (tile tid >> 6), threads < TM one scale each
    const int c0i = CPW * w, t4 = c0i >> 3, kc0 = c0i & 7;
    const int64_t sm0 = m0 + 32 * t4 + (lane & 31);
    const int64_t sm = sm0 < M ? sm0 : M - 1;
    const v4i *ag = reinterpret_cast<const v4i *>(q + sm * K) + (lane >> 5) + 2 * kc0;  // + 16 b + 2 r
    const int64_t ss0 = m0 + 32 * (tid >> 6) + (lane & 31);  // msum operand row (threads < 2 TM)
    const int64_t srow = ss0 < M ? ss0 : M - 1;
    const v4i *sg2 = reinterpret_cast<const v4i *>(sj + srow * nb * 16) + (lane >> 5);  // + 2 b
    const int64_t dm0 = m0 + (tid & (TM - 1));
    const float *dg = d8 + (dm0 < M ? dm0 : M - 1) * nb;
    v4i sa[CPW], ss = (v4i){0};
    float sd8 = 0.0f;
    auto fetch_a = [&](int b) {
#pragma unroll
        for (int r = 0; r < CPW; r++) sa[r] = ag[16 * b + 2 * r];
        if (tid < 2 * TM) ss = sg2[2 * b];
        if (tid < TM) sd8 = dg[b];
    };
    auto put_a = [&](int buf) {
        uint8_t *st = lds + buf * STAGE;
        v4i *ad = reinterpret_cast<v4i *>(st + (8 * t4 + kc0) * 1024) + lane;
#pragma unroll
        for (int r = 0; r < CPW; r++) ad[64 * r] = sa[r];
        if (tid < 2 * TM) reinterpret_cast<v4i *>(st + ABYTES)[tid] = ss;
        if (tid < TM) reinterpret_cast<float *>(st + ABYTES + SBYTES)[tid] = sd8;
    };

    // this wave's weight rows: lane l holds row 32w + l%32, code bytes 64 (l/32) + 16g .. +15 of each block
    // (elements 16 (l/32) .. +15 of sub-blocks 2g (low nibbles) and 2g+1 (high nibbles))
    const int nloc = 32 * w + (lane & 31);
    const int64_t wrow = row0 + ((n0 + nloc) < N ? (n0 + nloc) : N - 1);
    const uint4 *hq = reinterpret_cast<const uint4 *>(p.aux) + wrow * nb;
    const uint4 *qq = reinterpret_cast<const uint4 *>(p.qs) + wrow * nb * 8 + 4 * (lane >> 5);  // + 8 b + g
    uint4 wh, wq[4];
    auto fetch_w = [&](int b) {
        wh = hq[b];
#pragma unroll
        for (int g = 0; g < 4; g++) wq[g] = qq[8 * b + g];
    };

    fetch_a(0);
    fetch_w(0);
    put_a(0);
    if (nb > 1) fetch_a(1);
    __syncthreads();

    float accf[MT][16];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) accf[t][v] = 0.0f;

    for (int b = 0; b < nb; b++) {
        const uint8_t *st = lds + (b & 1) * STAGE;
        // weight block b: scales, then the next block's bytes are requested
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(wh.y, wh.z, wh.w, sc_lo, sc_hi, m_lo, m_hi);
        const float dd = f16_to_f32((uint16_t)(wh.x & 0xFFFF)), dm = f16_to_f32((uint16_t)(wh.x >> 16));
        uint4 cq[4] = {wq[0], wq[1], wq[2], wq[3]};
        const uint32_t mlo = m_lo, mhi = m_hi;
        if (b + 1 < nb) fetch_w(b + 1);

        v16i c0[MT], c1[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) {
            c0[t] = (v16i){0};
            c1[t] = (v16i){0};
        }
        const v4i *ar = reinterpret_cast<const v4i *>(st) + lane;  // tile t: + 512 t, chunk kc: + 64 kc
#pragma unroll
        for (int kc = 0; kc < 8; kc++) {
            const uint4 raw = cq[kc >> 1];
            const uint4 nib = (kc & 1) ? make_uint4((raw.x >> 4) & 0x0F0F0F0Fu, (raw.y >> 4) & 0x0F0F0F0Fu,
                                                    (raw.z >> 4) & 0x0F0F0F0Fu, (raw.w >> 4) & 0x0F0F0F0Fu)
                                       : make_uint4(raw.x & 0x0F0F0F0Fu, raw.y & 0x0F0F0F0Fu, raw.z & 0x0F0F0F0Fu,
                                                    raw.w & 0x0F0F0F0Fu);
            const uint32_t sc = ((kc < 4 ? sc_lo : sc_hi) >> (8 * (kc & 3))) & 0xFF;
            const v4i b0 = mul16(nib, sc & 7), b1 = mul16(nib, sc >> 3);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i a = ar[512 * t + 64 * kc];
                c0[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b0, c0[t], 0, 0, 0);
                c1[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b1, c1[t], 0, 0, 0);
            }
        }
        // stage block b + 1 into the other buffer (last read before the previous barrier), request block b + 2
        if (b + 1 < nb) {
            put_a((b + 1) & 1);
            if (b + 2 < nb) fetch_a(b + 2);
        }
        // msum B operand of this lane's row: [64 m_0..7 | m_0..7] (lanes < 32 hold k 0..7, lanes >= 32 k 8..15)
        const uint32_t mul = (lane >> 5) ? 1u : 64u;
        const v8h bmv = __builtin_bit_cast(
            v8h, make_uint4(pack_h2(mul * (mlo & 0xFF), mul * ((mlo >> 8) & 0xFF)),
                            pack_h2(mul * ((mlo >> 16) & 0xFF), mul * (mlo >> 24)),
                            pack_h2(mul * (mhi & 0xFF), mul * ((mhi >> 8) & 0xFF)),
                            pack_h2(mul * ((mhi >> 16) & 0xFF), mul * (mhi >> 24))));
        const float *d8s = reinterpret_cast<const float *>(st + ABYTES + SBYTES);
        // per-block epilogue in the reference's rounding order
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const v8h am = *reinterpret_cast<const v8h *>(st + ABYTES + t * 1024 + 16 * lane);
            const v16f cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bmv, (v16f){0}, 0, 0, 0);
#pragma unroll
            for (int v4 = 0; v4 < 4; v4++) {
                const float4 s8 = *reinterpret_cast<const float4 *>(d8s + 32 * t + 8 * v4 + 4 * (lane >> 5));
                const float s8v[4] = {s8.x, s8.y, s8.z, s8.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int v = 4 * v4 + r;
                    const int isum = c0[t][v] + 8 * c1[t][v];
                    const float tt = (dd * (float)isum) - (dm * cm[v]);
                    accf[t][v] = accf[t][v] + tt * s8v[r];
                }
            }
        }
        __syncthreads();  // block b + 1 staged; nobody reads buffer b & 1 any more
    }

    const int64_t gn = n0 + nloc;
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int mloc = 32 * t + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            if (gn < N && rowstate[mloc] == 0) {
                float *o = c + (m0 + mloc) * N + gn;
                *o = ACC ? *o + accf[t][v] : accf[t][v];
            }
        }
    }
    // rows holding NaN/Inf take the exact fp32 path (quantGemv) on their own; rare
    if (!*anybad) return;
    for (int i = tid; i < TM * TN; i += THREADS) {
        const int ml = i / TN, nl = i % TN;
        const int64_t gn2 = n0 + nl;
        if (rowstate[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = exact_dot_row<kQ4K>(p, row0 + gn2, x + gm * K, K);
        float *o = c + gm * N + gn2;
        *o = ACC ? *o + v : v;
    }
}


template <int TM>
int run_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, int64_t M,
             bool acc, const int8_t *q, const float *d, const uint16_t *sj, const uint8_t *bad) {
    constexpr size_t lds = Tile<TM>::LDS;
    dim3 grid((unsigned)(((N + TN - 1) / TN) * ((M + TM - 1) / TM))), block(THREADS);
    static bool lds_set = false;  // more than 64 KB of dynamic LDS has to be allowed once per kernel
    if (!lds_set) {
        hipError_t e1 = hipFuncSetAttribute(reinterpret_cast<const void *>(&actq_mfma_q4k<true, TM>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        hipError_t e2 = hipFuncSetAttribute(reinterpret_cast<const void *>(&actq_mfma_q4k<false, TM>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e1 != hipSuccess) return hip_fail(ctx, e1, "actq_mfma: LDS size");
        if (e2 != hipSuccess) return hip_fail(ctx, e2, "actq_mfma: LDS size");
        lds_set = true;
    }
    if (acc)
        hipLaunchKernelGGL((actq_mfma_q4k<true, TM>), grid, block, lds, ctx->stream, w->planes(), N, row0, M, w->K, x, q, d,
                           sj, bad, c);
    else
        hipLaunchKernelGGL((actq_mfma_q4k<false, TM>), grid, block, lds, ctx->stream, w->planes(), N, row0, M, w->K, x, q,
                           d, sj, bad, c);
    return launch_check(ctx, "actq_mfma_q4k");
}

}  // namespace

int launch_actq_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     int64_t M, bool acc, const int8_t *q, const float *d, const uint16_t *sj, const uint8_t *bad) {
    if (w->dtype != kQ4K) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq_mfma: q4_k only");
    // row-tile height: TRHIP_ACTQ_TM (32 or 64) overrides the default
    static const int tm = [] {
        const char *e = getenv("TRHIP_ACTQ_TM");
        return (e && atoi(e) == 32) ? 32 : 64;
    }();
    if (tm == 32) return run_mfma<32>(ctx, w, row0, N, x, c, M, acc, q, d, sj, bad);
    return run_mfma<64>(ctx, w, row0, N, x, c, M, acc, q, d, sj, bad);
}

}  // namespace trhip
