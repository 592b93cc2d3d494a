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
#include "mfma_util.hpp"

#include <cfloat>
#include <cstdlib>

namespace trhip {
namespace {

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

// msum = sum_j S_j m_j with S_j = 64 Sh_j + Sl_j: one f16 MFMA over k = [Sh_0..7 | Sl_0..7] x [64 m_0..7 | m_0..7].
// Every product and partial sum is an integer below 2^24, so the fp32 result is msum exactly.
// FAST: the same integer sums with the two products and the accumulation fused (within 1e-4 of the exact result).
// S > 1 (FAST only): workgroup slice sl of a tile takes blocks [sl bps, sl bps + bps) and writes its partial tile; the
// workgroup that arrives last at the tile's counter adds the S partials in slice order (so the result does not
// depend on arrival order), writes c and returns the counter to zero, as rows16.hip does.
template <bool ACC, int TM, bool FAST>
__global__ __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(TM == 64 ? 2 : 3, TM == 64 ? 2 : 4))) void actq_mfma_q4k(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const int8_t *__restrict__ q, const float *__restrict__ d8, const uint16_t *__restrict__ sj,
    const uint8_t *__restrict__ bad_blk, float *__restrict__ c, int S, int bps, float *__restrict__ part,
    uint32_t *__restrict__ arrivals) {
    using T = Tile<TM>;
    __shared__ int lastflag;
    constexpr int MT = T::MT, ABYTES = T::ABYTES, SBYTES = T::SBYTES, STAGE = T::STAGE, CPW = T::CPW;
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowstate = reinterpret_cast<int *>(lds + 2 * STAGE);  // [TM] 0 ok, 1 NaN/Inf row, 2 outside M
    int *anybad = rowstate + TM;                                // some row of the tile is 1

    const int nb = (int)p.nb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    const int64_t tiles = ((M + TM - 1) / TM) * ((N + TN - 1) / TN);
    const int64_t tix = (int64_t)blockIdx.x % tiles;
    const int sl = (int)((int64_t)blockIdx.x / tiles);
    const int cb0 = sl * bps, cb1 = cb0 + bps < nb ? cb0 + bps : nb;  // this workgroup's blocks
    tile_of(tix, (M + TM - 1) / TM, (N + TN - 1) / TN, tmi, tni);
    const int64_t n0 = tni * TN, m0 = tmi * TM;
    tile_row_flags<TM, THREADS>(bad_blk, m0, M, nb, rowstate, anybad);

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

    fetch_a(cb0);
    fetch_w(cb0);
    put_a(0);
    if (cb0 + 1 < cb1) fetch_a(cb0 + 1);
    __syncthreads();

    float accf[MT][16];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) accf[t][v] = 0.0f;

    for (int b = cb0; b < cb1; b++) {
        const uint8_t *st = lds + ((b - cb0) & 1) * STAGE;
        // weight block b: scales, then the next block's bytes are requested
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(wh.y, wh.z, wh.w, sc_lo, sc_hi, m_lo, m_hi);
        const float dd = f16_to_f32((uint16_t)(wh.x & 0xFFFF)), dm = f16_to_f32((uint16_t)(wh.x >> 16));
        uint4 cq[4] = {wq[0], wq[1], wq[2], wq[3]};
        const uint32_t mlo = m_lo, mhi = m_hi;
        if (b + 1 < cb1) fetch_w(b + 1);

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
        if (b + 1 < cb1) {
            put_a((b + 1 - cb0) & 1);
            if (b + 2 < cb1) fetch_a(b + 2);
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
                    if (FAST) {
                        accf[t][v] = fmaf(fmaf(-dm, cm[v], dd * (float)isum), s8v[r], accf[t][v]);
                    } else {
                        const float tt = (dd * (float)isum) - (dm * cm[v]);
                        accf[t][v] = accf[t][v] + tt * s8v[r];
                    }
                }
            }
        }
        __syncthreads();  // block b + 1 staged; nobody reads buffer b & 1 any more
    }

    const int64_t gn = n0 + nloc;
    if (S == 1) {
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
    } else {
        // the slice's partial tile [TM][TN], passed between workgroups as agent-scope atomic stores and loads (the
        // L2 of each XCD does not hold them back); each thread's stores complete before the workgroup counts in
        float *pp = part + (tix * S + sl) * (int64_t)(TM * TN);
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int mloc = 32 * t + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                __hip_atomic_store(pp + mloc * TN + nloc, accf[t][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (tid == 0)
            lastflag = __hip_atomic_fetch_add(&arrivals[tix], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                       (uint32_t)(S - 1);
        __syncthreads();
        if (!lastflag) return;
        if (tid == 0) __hip_atomic_store(&arrivals[tix], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float *p0 = part + tix * S * (int64_t)(TM * TN);
        for (int i = tid; i < TM * TN; i += THREADS) {
            const int ml = i / TN, nl = i % TN;
            if (n0 + nl >= N || rowstate[ml] != 0) continue;
            float sv = __hip_atomic_load(p0 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (int k = 1; k < S; k++)
                sv = sv + __hip_atomic_load(p0 + k * (int64_t)(TM * TN) + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float *o = c + (m0 + ml) * N + (n0 + nl);
            *o = ACC ? *o + sv : sv;
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
             bool acc, const int8_t *q, const float *d, const uint16_t *sj, const uint8_t *bad, bool fast, int S) {
    constexpr size_t lds = Tile<TM>::LDS;
    const int64_t tiles = ((N + TN - 1) / TN) * ((M + TM - 1) / TM), nb = w->nb;
    if (!fast || S < 1) S = 1;  // the exact mode adds the blocks in order
    if (S > nb) S = (int)nb;
    const int bps = (int)((nb + S - 1) / S);
    S = (int)((nb + bps - 1) / bps);
    float *part = nullptr;
    if (S > 1) {
        if (tiles > trhip_ctx::kArrivalSlots || !ctx->arrivals) S = 1;
        int st = TRHIP_OK;
        if (S > 1 && !(part = static_cast<float *>(workspace2(ctx, (size_t)(tiles * S * TM * TN) * sizeof(float), &st))))
            return st;
    }
    dim3 grid((unsigned)(tiles * S)), block(THREADS);
    static_assert(lds <= 64 * 1024, "below 64 KB of LDS no launch attribute is needed");
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, lds, ctx->stream, w->planes(), N, row0, M, w->K, x, q, d, sj, bad, c, S,
                           S > 1 ? bps : (int)nb, part, ctx->arrivals);
        return launch_check(ctx, "actq_mfma_q4k");
    };
    if (fast) return acc ? go(&actq_mfma_q4k<true, TM, true>) : go(&actq_mfma_q4k<false, TM, true>);
    return acc ? go(&actq_mfma_q4k<true, TM, false>) : go(&actq_mfma_q4k<false, TM, false>);
}

// ---- Fast (tolerance) M > 1 path for q4_k: fp32 activations as three int8 digit planes ----
//
// The reference's GPU backend runs M > 1 as dequantized tiles through a float GEMM (gpu/backend_quant.go:43-134):
// a tolerance path. Here each 256-wide block b of activation row m is put on a fixed-point grid,
//   max|x| = f 2^E (f in [0.5, 1), E one higher when f > 127/128),  X_i = rint(x_i 2^(23-E)),  |X_i| <= 127 2^16,
//   X = D0 + 256 D1 + 65536 D2  with balanced digits D0, D1 in [-128, 127] and D2 in [-128, 127],
// so that with q4_k weights y = d sc_j q - dmin m_j,
//   sum_i x_i y_i ~= 2^(E-23) (d isum - dmin msum),
//   isum = sum_t 256^t sum_i (sc q)_i D_t,i    three int8 MFMA accumulations per scale half, exact in int32,
//   msum = sum_j m_j XS_j,  XS_j = sum_{i in j} X_i = P0 + 512 P1 + 2^18 P2 (f16-exact parts, |P2| <= 1016), one
// f16 MFMA pair. Besides the grid (2^-23 to 2^-22 of the block's largest |x|) only the fp32 epilogue rounds, within
// the 1e-4 tolerance of the fast mode.
// Rows holding NaN/Inf are computed with exact float dot products instead, as the act-quant path does.

constexpr int FM_TM = 32, FM_TN = 128, FM_THREADS = 256;
constexpr int FM_DIGIT = 8 * 1024;               // one digit plane of a 32-row block tile, MFMA lane order
constexpr int FM_STAGE = 3 * FM_DIGIT + 2 * 1024 + FM_TM * 4;  // digits, msum A operands, exponents
constexpr size_t FM_LDS = 2 * FM_STAGE + (FM_TM + 1) * sizeof(int);

// Slot of 16-byte A piece (row r < 32, piece j < 16 of the block's 256 bytes) in a digit plane: chunk kc = j / 2
// of 64 lanes, lane 32 (j % 2) + r, with the low four bits xor-ed by j so that the 16 pieces of one row (written
// by 16 consecutive threads) fall on distinct LDS banks; the MFMA read of chunk kc by lane l is slot
// 64 kc + (l ^ (2 kc + l / 32) % 16), a permutation of that chunk's 64 slots.
__device__ __forceinline__ int fm_slot(int r, int j) { return 64 * (j >> 1) + ((32 * (j & 1) + r) ^ (j & 15)); }

// One wave per (row m, block b): exponent, digit planes, the f16 parts of the sub-block sums, and a NaN/Inf flag.
__global__ __launch_bounds__(256) void digits_q4k_kernel(const float *__restrict__ x, int64_t M, int64_t K,
                                                         int8_t *__restrict__ dg, int *__restrict__ ex,
                                                         uint16_t *__restrict__ xsp, uint8_t *__restrict__ bad) {
    const int lane = threadIdx.x & 63;
    const int64_t nb = K / 256;
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= M * nb) return;  // wave-uniform
    const int64_t m = gw / nb, b = gw % nb;
    const float4 v = reinterpret_cast<const float4 *>(x + m * K + 256 * b)[lane];
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    const bool fin = (fabsf(v.x) <= FLT_MAX) && (fabsf(v.y) <= FLT_MAX) && (fabsf(v.z) <= FLT_MAX) &&
                     (fabsf(v.w) <= FLT_MAX);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const bool allfin = __all(fin);
    int E = 0;
    if (allfin && amax > 0.0f && frexpf(amax, &E) > 127.0f / 128.0f) E += 1;  // keeps |X| <= 127 2^16
    const float xv[4] = {v.x, v.y, v.z, v.w};
    int X[4];
    uint32_t d0 = 0, d1 = 0, d2 = 0;
    int xs = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        X[i] = allfin ? (int)rintf(ldexpf(xv[i], 23 - E)) : 0;
        const int a0 = (int)(int8_t)(X[i] & 0xFF), r1 = (X[i] - a0) >> 8;
        const int a1 = (int)(int8_t)(r1 & 0xFF), a2 = (r1 - a1) >> 8;
        d0 |= (uint32_t)(a0 & 0xFF) << (8 * i);
        d1 |= (uint32_t)(a1 & 0xFF) << (8 * i);
        d2 |= (uint32_t)(a2 & 0xFF) << (8 * i);
        xs += X[i];
    }
    uint32_t *row = reinterpret_cast<uint32_t *>(dg + m * K + 256 * b) + lane;
    const int64_t plane = M * K / 4;  // words per digit plane
    row[0] = d0;
    row[plane] = d1;
    row[2 * plane] = d2;
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) xs += __shfl_xor(xs, o);  // sub-block j = lane / 8
    if ((lane & 7) == 0) {
        const int j = lane >> 3;
        const int p0 = ((xs + 256) & 511) - 256, r = (xs - p0) >> 9;
        const int p1 = ((r + 256) & 511) - 256, p2 = (r - p1) >> 9;
        uint16_t *o = xsp + (m * nb + b) * 24;
        o[j] = __builtin_bit_cast(uint16_t, (_Float16)(float)p0);
        o[8 + j] = __builtin_bit_cast(uint16_t, (_Float16)(float)p1);
        o[16 + j] = __builtin_bit_cast(uint16_t, (_Float16)(float)p2);
    }
    if (lane == 0) {
        ex[m * nb + b] = E - 23;
        bad[m * nb + b] = allfin ? 0 : 1;
    }
}

// Workgroup (tile, slice): 32 activation rows x 128 weight rows over blocks [bps s, bps s + bps). Wave w owns weight
// rows 32 w .. +31 (lane l: row l % 32, as in actq_mfma_q4k). A block's digit planes, msum operands and exponents
// are staged in LDS (double-buffered, coalesced: 16 consecutive threads read one row's 256 bytes).
template <bool ACC>
__global__ __launch_bounds__(FM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void fastm_mfma_q4k(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const int8_t *__restrict__ dg, const int *__restrict__ ex, const uint16_t *__restrict__ xsp,
    const uint8_t *__restrict__ bad, int64_t bps, float *__restrict__ c, float *__restrict__ partial) {
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowbad = reinterpret_cast<int *>(lds + 2 * FM_STAGE);  // [FM_TM] 0 ok, 1 NaN/Inf row, 2 outside M
    int *anybad = rowbad + FM_TM;
    const int nb = (int)p.nb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + FM_TM - 1) / FM_TM, (N + FM_TN - 1) / FM_TN, tmi, tni);
    const int64_t n0 = tni * FM_TN, m0 = tmi * FM_TM;
    const int b0 = (int)(blockIdx.y * bps), b1 = (int)((blockIdx.y + 1) * bps < nb ? (blockIdx.y + 1) * bps : nb);
    tile_row_flags<FM_TM, FM_THREADS>(bad, m0, M, nb, rowbad, anybad);

    // staging roles: digit pieces P = tid + 256 i (i < 2) of each plane: row P / 16, piece P % 16; threads < 128 also
    // stage one msum operand piece (row tid % 32, part pair tid / 32 < 2 ... see below), threads < 32 one exponent
    const int64_t plane = M * K;
    int8_t const *dsrc[2];
    int dslot[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int P = tid + 256 * i, r = P >> 4, j = P & 15;
        const int64_t gm = m0 + r < M ? m0 + r : M - 1;
        dsrc[i] = dg + gm * K + 16 * j;
        dslot[i] = fm_slot(r, j);
    }
    // msum A operands, 32x32x16 f16 layout (lane l: row l % 32, k 8 (l / 32) .. +7): operand 0 = [P0 | P1],
    // operand 1 = [P2 | 0]; thread tid < 128 stages 16 bytes: operand tid / 64, lane tid % 64
    const int sr = tid & 31, sop = (tid >> 6) & 1, shalf = (tid >> 5) & 1;
    const int64_t sgm = m0 + sr < M ? m0 + sr : M - 1;
    const uint16_t *ssrc = xsp + sgm * nb * 24 + 8 * (2 * sop + shalf);  // + 24 b; part 3 (sop 1, half 1) is zero
    const int64_t egm = m0 + (tid & 31) < M ? m0 + (tid & 31) : M - 1;
    v4i sa[2][3];
    v4i ss = (v4i){0};
    int se = 0;
    auto fetch_a = [&](int b) {
#pragma unroll
        for (int t = 0; t < 3; t++)
#pragma unroll
            for (int i = 0; i < 2; i++) sa[i][t] = *reinterpret_cast<const v4i *>(dsrc[i] + t * plane + 256 * (int64_t)b);
        if (tid < 128) ss = (sop == 1 && shalf == 1) ? (v4i){0} : *reinterpret_cast<const v4i *>(ssrc + 24 * (int64_t)b);
        if (tid < FM_TM) se = ex[egm * nb + b];
    };
    auto put_a = [&](int buf) {
        uint8_t *st = lds + buf * FM_STAGE;
#pragma unroll
        for (int t = 0; t < 3; t++)
#pragma unroll
            for (int i = 0; i < 2; i++) reinterpret_cast<v4i *>(st + t * FM_DIGIT)[dslot[i]] = sa[i][t];
        if (tid < 128) reinterpret_cast<v4i *>(st + 3 * FM_DIGIT)[tid] = ss;
        if (tid < FM_TM) reinterpret_cast<int *>(st + 3 * FM_DIGIT + 2048)[tid] = se;
    };

    const int nloc = 32 * w + (lane & 31);
    const int64_t wrow = row0 + ((n0 + nloc) < N ? (n0 + nloc) : N - 1);
    const uint4 *hq = reinterpret_cast<const uint4 *>(p.aux) + wrow * nb;
    const uint4 *qq = reinterpret_cast<const uint4 *>(p.qs) + wrow * nb * 8 + 4 * (lane >> 5);
    uint4 wh, wq[4];
    auto fetch_w = [&](int b) {
        wh = hq[b];
#pragma unroll
        for (int g = 0; g < 4; g++) wq[g] = qq[8 * b + g];
    };

    float accf[16];
#pragma unroll
    for (int v = 0; v < 16; v++) accf[v] = 0.0f;
    if (b0 < b1) {
        fetch_a(b0);
        fetch_w(b0);
        put_a(0);
        if (b0 + 1 < b1) fetch_a(b0 + 1);
    }
    __syncthreads();

    for (int b = b0; b < b1; b++) {
        const uint8_t *st = lds + ((b - b0) & 1) * FM_STAGE;
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(wh.y, wh.z, wh.w, sc_lo, sc_hi, m_lo, m_hi);
        const float dd = f16_to_f32((uint16_t)(wh.x & 0xFFFF)), dm = f16_to_f32((uint16_t)(wh.x >> 16));
        const uint4 cq[4] = {wq[0], wq[1], wq[2], wq[3]};
        const uint32_t mlo = m_lo, mhi = m_hi;
        if (b + 1 < b1) fetch_w(b + 1);

        v16i c0[3], c1[3];
#pragma unroll
        for (int t = 0; t < 3; t++) {
            c0[t] = (v16i){0};
            c1[t] = (v16i){0};
        }
#pragma unroll
        for (int kc = 0; kc < 8; kc++) {
            const uint4 raw = cq[kc >> 1];
            const uint4 nib = (kc & 1) ? make_uint4((raw.x >> 4) & 0x0F0F0F0Fu, (raw.y >> 4) & 0x0F0F0F0Fu,
                                                    (raw.z >> 4) & 0x0F0F0F0Fu, (raw.w >> 4) & 0x0F0F0F0Fu)
                                       : make_uint4(raw.x & 0x0F0F0F0Fu, raw.y & 0x0F0F0F0Fu, raw.z & 0x0F0F0F0Fu,
                                                    raw.w & 0x0F0F0F0Fu);
            const uint32_t sc = ((kc < 4 ? sc_lo : sc_hi) >> (8 * (kc & 3))) & 0xFF;
            const v4i wb0 = mul16(nib, sc & 7), wb1 = mul16(nib, sc >> 3);
            const int slot = 64 * kc + (lane ^ ((2 * kc + (lane >> 5)) & 15));
#pragma unroll
            for (int t = 0; t < 3; t++) {
                const v4i a = reinterpret_cast<const v4i *>(st + t * FM_DIGIT)[slot];
                c0[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, wb0, c0[t], 0, 0, 0);
                c1[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, wb1, c1[t], 0, 0, 0);
            }
        }
        float fs[16];  // sum_t 128^t isum_t
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float f0 = (float)(c0[0][v] + 8 * c1[0][v]), f1 = (float)(c0[1][v] + 8 * c1[1][v]),
                        f2 = (float)(c0[2][v] + 8 * c1[2][v]);
            fs[v] = fmaf(65536.0f, f2, fmaf(256.0f, f1, f0));
        }
        if (b + 1 < b1) {
            put_a((b + 1 - b0) & 1);
            if (b + 2 < b1) fetch_a(b + 2);
        }
        // msum B operands of this lane's weight row: [m_0..7 | 512 m_0..7] and [m_0..7 | 0]
        const uint32_t mul = (lane >> 5) ? 512u : 1u;
        const v8h bm0 = __builtin_bit_cast(
            v8h, make_uint4(pack_h2(mul * (mlo & 0xFF), mul * ((mlo >> 8) & 0xFF)),
                            pack_h2(mul * ((mlo >> 16) & 0xFF), mul * (mlo >> 24)),
                            pack_h2(mul * (mhi & 0xFF), mul * ((mhi >> 8) & 0xFF)),
                            pack_h2(mul * ((mhi >> 16) & 0xFF), mul * (mhi >> 24))));
        const v8h bm1 = (lane >> 5) ? (v8h){0, 0, 0, 0, 0, 0, 0, 0}
                                    : __builtin_bit_cast(v8h, make_uint4(pack_h2(mlo & 0xFF, (mlo >> 8) & 0xFF),
                                                                         pack_h2((mlo >> 16) & 0xFF, mlo >> 24),
                                                                         pack_h2(mhi & 0xFF, (mhi >> 8) & 0xFF),
                                                                         pack_h2((mhi >> 16) & 0xFF, mhi >> 24)));
        const v8h am0 = *reinterpret_cast<const v8h *>(st + 3 * FM_DIGIT + 16 * lane);
        const v8h am1 = *reinterpret_cast<const v8h *>(st + 3 * FM_DIGIT + 1024 + 16 * lane);
        const v16f cm0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(am0, bm0, (v16f){0}, 0, 0, 0);
        const v16f cm1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(am1, bm1, (v16f){0}, 0, 0, 0);
        const int *exs = reinterpret_cast<const int *>(st + 3 * FM_DIGIT + 2048);
#pragma unroll
        for (int v4 = 0; v4 < 4; v4++) {
            const int4 e4 = *reinterpret_cast<const int4 *>(exs + 8 * v4 + 4 * (lane >> 5));
            const int ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int v = 4 * v4 + r;
                const float ms = fmaf(262144.0f, cm1[v], cm0[v]);
                accf[v] = accf[v] + ldexpf(fmaf(dd, fs[v], -(dm * ms)), ev[r]);
            }
        }
        __syncthreads();  // block b + 1 staged; nobody reads buffer (b - b0) & 1 any more
    }

    const int64_t gn = n0 + nloc;
    float *dst = partial ? partial + (int64_t)blockIdx.y * M * N : c;
    const bool acc_c = ACC && partial == nullptr;
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int mloc = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (gn < N && rowbad[mloc] == 0) {
            float *o = dst + (m0 + mloc) * N + gn;
            *o = acc_c ? *o + accf[v] : accf[v];
        }
    }
    // rows holding NaN/Inf: exact float dot products over the whole row, by slice 0 (the other slices add zero)
    if (!*anybad) return;
    for (int i = tid; i < FM_TM * FM_TN; i += FM_THREADS) {
        const int ml = i / FM_TN, nl = i % FM_TN;
        const int64_t gn2 = n0 + nl;
        if (rowbad[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = blockIdx.y == 0 ? exact_dot_row<kQ4K>(p, row0 + gn2, x + gm * K, K) : 0.0f;
        float *o = dst + gm * N + gn2;
        *o = acc_c ? *o + v : v;
    }
}

// The same for at most 16 activation rows, on 16-row tiles: v_mfma_i32_16x16x64_i8 and v_mfma_f32_16x16x32_f16
// (lane l: row / column l % 16, k-slice l / 16 of 16 bytes / 8 halves; result register v of lane l: row 4 (l / 16) + v,
// column l % 16, both checked on the device). Wave w owns weight rows 32 w .. +31 as two 16-column tiles; for 64-wide
// chunk c of a block, lane l's B operand is elements 16 (l / 16) .. +15 of chunk c, i.e. of sub-block 2 c + l / 32,
// held in the lane-sliced q4_k bytes 64 ((l / 16) & 1) + 16 c .. +15 (low nibbles for l < 32, high for l >= 32).
constexpr int F16_TM = 16;
constexpr int F16_DIGIT = 4 * 1024;                              // one digit plane of a 16-row block tile
constexpr int F16_STAGE = 3 * F16_DIGIT + 2 * 1024 + F16_TM * 4;  // digits, msum A operands, exponents
constexpr size_t F16_LDS = 2 * F16_STAGE + (F16_TM + 1) * sizeof(int);

// Slot of 16-byte A piece (row r < 16, piece j < 16) in a 16-row digit plane: chunk j / 4 of 64 lanes, lane
// 16 (j % 4) + r, low four bits xor-ed by j (the 16 pieces of a row land on distinct banks); the read of chunk c by
// lane l is slot 64 c + (l ^ (4 c + l / 16) % 16).
__device__ __forceinline__ int f16_slot(int r, int j) { return 64 * (j >> 2) + ((16 * (j & 3) + r) ^ (j & 15)); }

template <bool ACC>
__global__ __launch_bounds__(FM_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void fastm16_mfma_q4k(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const int8_t *__restrict__ dg, const int *__restrict__ ex, const uint16_t *__restrict__ xsp,
    const uint8_t *__restrict__ bad, int64_t bps, float *__restrict__ c, float *__restrict__ partial) {
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowbad = reinterpret_cast<int *>(lds + 2 * F16_STAGE);
    int *anybad = rowbad + F16_TM;
    const int nb = (int)p.nb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + F16_TM - 1) / F16_TM, (N + FM_TN - 1) / FM_TN, tmi, tni);
    const int64_t n0 = tni * FM_TN, m0 = tmi * F16_TM;
    const int b0 = (int)(blockIdx.y * bps), b1 = (int)((blockIdx.y + 1) * bps < nb ? (blockIdx.y + 1) * bps : nb);
    tile_row_flags<F16_TM, FM_THREADS>(bad, m0, M, nb, rowbad, anybad);

    // staging: digit piece tid of each plane (row tid / 16, piece tid % 16); threads < 128 one msum operand piece
    // (operand tid / 64: [P0 | P1 | 0 | 0] or [P2 | 0 | 0 | 0], lane tid % 64: row lane % 16, k-group lane / 16);
    // threads < 16 one exponent
    const int64_t plane = M * K;
    const int dr = tid >> 4, dj = tid & 15;
    const int8_t *dsrc = dg + (m0 + dr < M ? m0 + dr : M - 1) * K + 16 * dj;
    const int dslot = f16_slot(dr, dj);
    const int sl = tid & 63, sop = (tid >> 6) & 1, sgrp = sl >> 4;  // k-group of 8 halves
    const int64_t sgm = m0 + (sl & 15) < M ? m0 + (sl & 15) : M - 1;
    const bool sval = sop == 0 ? sgrp < 2 : sgrp == 0;  // which groups carry parts
    const uint16_t *ssrc = xsp + sgm * nb * 24 + 8 * (sop == 0 ? sgrp : 2);  // + 24 b
    const int64_t egm = m0 + (tid & 15) < M ? m0 + (tid & 15) : M - 1;
    v4i sa[3];
    v4i ss = (v4i){0};
    int se = 0;
    auto fetch_a = [&](int b) {
#pragma unroll
        for (int t = 0; t < 3; t++) sa[t] = *reinterpret_cast<const v4i *>(dsrc + t * plane + 256 * (int64_t)b);
        if (tid < 128) ss = sval ? *reinterpret_cast<const v4i *>(ssrc + 24 * (int64_t)b) : (v4i){0};
        if (tid < F16_TM) se = ex[egm * nb + b];
    };
    auto put_a = [&](int buf) {
        uint8_t *st = lds + buf * F16_STAGE;
#pragma unroll
        for (int t = 0; t < 3; t++) reinterpret_cast<v4i *>(st + t * F16_DIGIT)[dslot] = sa[t];
        if (tid < 128) reinterpret_cast<v4i *>(st + 3 * F16_DIGIT)[tid] = ss;
        if (tid < F16_TM) reinterpret_cast<int *>(st + 3 * F16_DIGIT + 2048)[tid] = se;
    };

    // weights: lane l, tile t: row 32 w + 16 t + l % 16, bytes 64 ((l / 16) & 1) .. +63 of each block
    const uint4 *hq[2], *qq[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int nl = 32 * w + 16 * t + (lane & 15);
        const int64_t wrow = row0 + ((n0 + nl) < N ? (n0 + nl) : N - 1);
        hq[t] = reinterpret_cast<const uint4 *>(p.aux) + wrow * nb;
        qq[t] = reinterpret_cast<const uint4 *>(p.qs) + wrow * nb * 8 + 4 * ((lane >> 4) & 1);
    }
    uint4 wh[2], wq[2][4];
    auto fetch_w = [&](int b) {
#pragma unroll
        for (int t = 0; t < 2; t++) {
            wh[t] = hq[t][b];
#pragma unroll
            for (int g = 0; g < 4; g++) wq[t][g] = qq[t][8 * b + g];
        }
    };

    float accf[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) accf[t][v] = 0.0f;
    if (b0 < b1) {
        fetch_a(b0);
        fetch_w(b0);
        put_a(0);
        if (b0 + 1 < b1) fetch_a(b0 + 1);
    }
    __syncthreads();

    const int hi = lane >> 5;  // this lane's sub-blocks are 2 c + hi: high nibbles for hi = 1
    for (int b = b0; b < b1; b++) {
        const uint8_t *st = lds + ((b - b0) & 1) * F16_STAGE;
        uint32_t scv[2][4];  // scale byte of sub-block 2 c + hi, per tile and chunk
        uint32_t mv[2][2];   // the tile rows' m_0..7 (lo, hi words)
        float dd[2], dm[2];
        uint4 cq[2][4];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            uint32_t sc_lo, sc_hi, m_lo, m_hi;
            q4k_scales(wh[t].y, wh[t].z, wh[t].w, sc_lo, sc_hi, m_lo, m_hi);
            dd[t] = f16_to_f32((uint16_t)(wh[t].x & 0xFFFF));
            dm[t] = f16_to_f32((uint16_t)(wh[t].x >> 16));
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                const int j = 2 * cc + hi;
                scv[t][cc] = ((j < 4 ? sc_lo : sc_hi) >> (8 * (j & 3))) & 0xFF;
            }
            mv[t][0] = m_lo;
            mv[t][1] = m_hi;
#pragma unroll
            for (int g = 0; g < 4; g++) cq[t][g] = wq[t][g];
        }
        if (b + 1 < b1) fetch_w(b + 1);

        v4i c0[2][3], c1[2][3];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int d = 0; d < 3; d++) {
                c0[t][d] = (v4i){0, 0, 0, 0};
                c1[t][d] = (v4i){0, 0, 0, 0};
            }
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const int slot = 64 * cc + (lane ^ ((4 * cc + (lane >> 4)) & 15));
            v4i a[3];
#pragma unroll
            for (int d = 0; d < 3; d++) a[d] = reinterpret_cast<const v4i *>(st + d * F16_DIGIT)[slot];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint4 raw = cq[t][cc];
                const uint4 nib = hi ? make_uint4((raw.x >> 4) & 0x0F0F0F0Fu, (raw.y >> 4) & 0x0F0F0F0Fu,
                                                  (raw.z >> 4) & 0x0F0F0F0Fu, (raw.w >> 4) & 0x0F0F0F0Fu)
                                     : make_uint4(raw.x & 0x0F0F0F0Fu, raw.y & 0x0F0F0F0Fu, raw.z & 0x0F0F0F0Fu,
                                                  raw.w & 0x0F0F0F0Fu);
                const uint32_t sc = scv[t][cc];
                const v4i wb0 = mul16(nib, sc & 7), wb1 = mul16(nib, sc >> 3);
#pragma unroll
                for (int d = 0; d < 3; d++) {
                    c0[t][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[d], wb0, c0[t][d], 0, 0, 0);
                    c1[t][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[d], wb1, c1[t][d], 0, 0, 0);
                }
            }
        }
        float fs[2][4];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float f0 = (float)(c0[t][0][v] + 8 * c1[t][0][v]), f1 = (float)(c0[t][1][v] + 8 * c1[t][1][v]),
                            f2 = (float)(c0[t][2][v] + 8 * c1[t][2][v]);
                fs[t][v] = fmaf(65536.0f, f2, fmaf(256.0f, f1, f0));
            }
        if (b + 1 < b1) {
            put_a((b + 1 - b0) & 1);
            if (b + 2 < b1) fetch_a(b + 2);
        }
        // msum: A operands [P0 | P1 | 0 | 0] and [P2 | 0 | 0 | 0] (k-groups of 8); B of this lane's column,
        // k-group l / 16: [m_0..7 | 512 m_0..7 | 0 | 0] and [m_0..7 | 0 | 0 | 0]
        const v8h am0 = *reinterpret_cast<const v8h *>(st + 3 * F16_DIGIT + 16 * lane);
        const v8h am1 = *reinterpret_cast<const v8h *>(st + 3 * F16_DIGIT + 1024 + 16 * lane);
        const int grp = lane >> 4;
        const int *exs = reinterpret_cast<const int *>(st + 3 * F16_DIGIT + 2048);
        const int4 e4 = *reinterpret_cast<const int4 *>(exs + 4 * grp);
        const int ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint32_t mlo = mv[t][0], mhi = mv[t][1];
            const uint32_t mul = grp == 1 ? 512u : 1u;
            const v8h mj = __builtin_bit_cast(
                v8h, make_uint4(pack_h2(mul * (mlo & 0xFF), mul * ((mlo >> 8) & 0xFF)),
                                pack_h2(mul * ((mlo >> 16) & 0xFF), mul * (mlo >> 24)),
                                pack_h2(mul * (mhi & 0xFF), mul * ((mhi >> 8) & 0xFF)),
                                pack_h2(mul * ((mhi >> 16) & 0xFF), mul * (mhi >> 24))));
            const v8h zero = (v8h){0, 0, 0, 0, 0, 0, 0, 0};
            const v8h bm0 = grp < 2 ? mj : zero, bm1 = grp == 0 ? mj : zero;
            const v4f cm0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(am0, bm0, (v4f){0, 0, 0, 0}, 0, 0, 0);
            const v4f cm1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(am1, bm1, (v4f){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float ms = fmaf(262144.0f, cm1[v], cm0[v]);
                accf[t][v] = accf[t][v] + ldexpf(fmaf(dd[t], fs[t][v], -(dm[t] * ms)), ev[v]);
            }
        }
        __syncthreads();
    }

    float *dst = partial ? partial + (int64_t)blockIdx.y * M * N : c;
    const bool acc_c = ACC && partial == nullptr;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int64_t gn = n0 + 32 * w + 16 * t + (lane & 15);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int mloc = 4 * (lane >> 4) + v;
            if (gn < N && rowbad[mloc] == 0) {
                float *o = dst + (m0 + mloc) * N + gn;
                *o = acc_c ? *o + accf[t][v] : accf[t][v];
            }
        }
    }
    if (!*anybad) return;
    for (int i = tid; i < F16_TM * FM_TN; i += FM_THREADS) {
        const int ml = i / FM_TN, nl = i % FM_TN;
        const int64_t gn2 = n0 + nl;
        if (rowbad[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = blockIdx.y == 0 ? exact_dot_row<kQ4K>(p, row0 + gn2, x + gm * K, K) : 0.0f;
        float *o = dst + gm * N + gn2;
        *o = acc_c ? *o + v : v;
    }
}

// c[i] (+)= partial[0][i] + partial[1][i] + ... in slice order.
template <bool ACC>
__global__ void fm_sum_kernel(const float *__restrict__ partial, float *__restrict__ c, int64_t MN, int64_t ns) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += (int64_t)gridDim.x * blockDim.x) {
        float s = partial[i];
        for (int64_t k = 1; k < ns; k += 8) {  // up to eight loads in flight, added in slice order
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = k + u < ns ? partial[(k + u) * MN + i] : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (k + u < ns) s = s + v[u];
        }
        c[i] = ACC ? c[i] + s : s;
    }
}


// Fast M > 1 for q6_k (tolerance), on v_mfma_f32_16x16x32_f16. halves_kernel writes each activation row in
// 256-element chunks as x' = x * 2^-E (E from the chunk's largest |x|, so |x'| < 1) split into two f16 planes,
// hi = f16(x') * 2^11 (exact scaling) and lo = f16((x' - f16(x')) * 2^11): hi + lo holds x' * 2^11 to about 2^-23 of
// the chunk's largest element, and both terms stay in the normal f16 range. The codes q - 32 are exact small integers
// in f16 (built from their bytes as 0x6400 | byte = 1024 + byte, then one packed f16 subtraction), and
// sc = (sc & ~1) + (sc & 1) makes both weight planes (q - 32) (sc & ~1) (even, at most 4096 in magnitude) and
// (q - 32) (sc & 1) exact in f16, so every MFMA product is exact and one fp32 accumulator takes the whole block:
//   acc += d * D * 2^(E-11),  D = sum over the block of (hi + lo) (q - 32) sc
// Lane l holds 8 halves of row / column l % 16 at k-slice l / 16; result register v of lane l is row 4 (l / 16) + v,
// column l % 16. Rows of x holding NaN / Inf take exact float dot products, as in the q4_k kernels.
// Workgroup (tile, slice): 16 activation rows x 128 weight rows over blocks [bps s, bps s + bps); wave w owns weight
// rows 32 w .. +31 as two 16-column tiles. A block's two planes are staged in LDS (double-buffered) as 16-byte slots
// 64 s + l (step s, lane l), so every MFMA operand read is one conflict-free ds_read_b128.
// (The same scheme for q8_0 / q4_0, with a per-block scale FMA after each step, measured slower than the exact
// kernel at M = 2..16: 37-40 us against 25-38 us at 14336 x 4096; those dtypes run exact.)
constexpr int FH_PLANE = 8 * 1024;                   // one f16 plane of a 16-row chunk
constexpr int FH_STAGE = 2 * FH_PLANE + F16_TM * 4;  // hi, lo, exponents
constexpr size_t FH_LDS = 2 * FH_STAGE + (F16_TM + 1) * sizeof(int);

// Operand lane l of step s sits in slot fh_swz(l, s) of the step's 64: its row bits (l % 16) XOR 4 (l / 16) + s % 4.
// A wave's stage writes (two rows, all 32 pieces of each) then spread over every bank group, and the MFMA's reads of
// a step stay a permutation within each 16-lane group.
__device__ __forceinline__ int fh_swz(int l, int s) { return l ^ ((4 * (l >> 4) + (s & 3)) & 15); }

// One wave per (row m, chunk b): exponent, the two f16 planes and the NaN/Inf flag.
__global__ __launch_bounds__(256) void halves_kernel(const float *__restrict__ x, int64_t M, int64_t K,
                                                     uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                     int *__restrict__ ex, uint8_t *__restrict__ bad) {
    const int lane = threadIdx.x & 63;
    const int64_t nb = K / 256;
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= M * nb) return;  // wave-uniform
    const int64_t m = gw / nb, b = gw % nb;
    const float4 v = reinterpret_cast<const float4 *>(x + m * K + 256 * b)[lane];
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    const bool fin = (fabsf(v.x) <= FLT_MAX) && (fabsf(v.y) <= FLT_MAX) && (fabsf(v.z) <= FLT_MAX) &&
                     (fabsf(v.w) <= FLT_MAX);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const bool allfin = __all(fin);
    int E = 0;
    if (allfin && amax > 0.0f) frexpf(amax, &E);  // amax = f 2^E, f in [0.5, 1)
    const float xv[4] = {v.x, v.y, v.z, v.w};
    uint16_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float xs = allfin ? ldexpf(xv[i], -E) : 0.0f;  // |xs| < 1
        const _Float16 xh = (_Float16)xs;
        h[i] = __builtin_bit_cast(uint16_t, (_Float16)((float)xh * 2048.0f));
        l[i] = __builtin_bit_cast(uint16_t, (_Float16)((xs - (float)xh) * 2048.0f));
    }
    const int64_t o = (m * K + 256 * b) / 4 + lane;  // 4 halves per lane
    reinterpret_cast<uint2 *>(hi)[o] = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
    reinterpret_cast<uint2 *>(lo)[o] = make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    if (lane == 0) {
        ex[m * nb + b] = E - 11;
        bad[m * nb + b] = allfin ? 0 : 1;
    }
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
// (native vector types: HIP's uint2 / uint4 structs are copied through scratch memory when carried across loops)
struct Q6Regs {  // one 16-column tile's weight registers for one q6_k block
    u32x4 ql0, ql1, qh, sc;  // the lane's 32 ql bytes and 16 qh bytes (repacked k-slice ks), the 16 scales
    uint32_t d;
};

__device__ __forceinline__ void q6_load(Q6Regs &r, const Planes p, int64_t row, int64_t c, int ks) {
    const int64_t bi = row * p.nb + c;
    const u32x4 *ql = reinterpret_cast<const u32x4 *>(p.qs + bi * 128 + 32 * ks);
    r.ql0 = ql[0];
    r.ql1 = ql[1];
    r.qh = *reinterpret_cast<const u32x4 *>(p.aux + bi * 64 + 16 * ks);
    r.sc = *reinterpret_cast<const u32x4 *>(p.sc + bi * 16);
    r.d = p.d[bi];
}

// Bytes 0, 1 (hi = false) or 2, 3 of w as the f16 pair (1024 + byte0, 1024 + byte1): v_perm_b32 places each byte
// under 0x64, the f16 exponent of 1024.
__device__ __forceinline__ h2 f16_pair(uint32_t w, bool hi) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, hi ? 0x04030402u : 0x04010400u));
}

// The 8 codes of step s (32-element group k4 = s % 4 of half n = s / 4) at k-slice ks as exact f16 q - 32: ql words
// 4n + 2 (k4 & 1), qh words 2n.
__device__ __forceinline__ v8h q6_codes(const Q6Regs &r, int s) {
    const int n = s >> 2, k4 = s & 3;
    const uint32_t qw[8] = {r.ql0.x, r.ql0.y, r.ql0.z, r.ql0.w, r.ql1.x, r.ql1.y, r.ql1.z, r.ql1.w};
    const uint32_t hw[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    const int sh = k4 >= 2 ? 4 : 0;
    const uint32_t w0 = ((qw[4 * n + 2 * (k4 & 1)] >> sh) & 0x0F0F0F0Fu) | (((hw[2 * n] >> (2 * k4)) & 0x03030303u) << 4);
    const uint32_t w1 =
        ((qw[4 * n + 2 * (k4 & 1) + 1] >> sh) & 0x0F0F0F0Fu) | (((hw[2 * n + 1] >> (2 * k4)) & 0x03030303u) << 4);
    const h2 off = (h2){(_Float16)1056.0f, (_Float16)1056.0f};
    const h2 a = f16_pair(w0, false) - off, b = f16_pair(w0, true) - off;
    const h2 c = f16_pair(w1, false) - off, d = f16_pair(w1, true) - off;
    return (v8h){a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

template <bool ACC>
__global__ __launch_bounds__(FM_THREADS) __attribute__((amdgpu_waves_per_eu(3, 3))) void fastm16_q6k(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const uint16_t *__restrict__ xh, const uint16_t *__restrict__ xl, const int *__restrict__ ex,
    const uint8_t *__restrict__ bad, int64_t bps, float *__restrict__ c, float *__restrict__ partial) {
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowbad = reinterpret_cast<int *>(lds + 2 * FH_STAGE);
    int *anybad = rowbad + F16_TM;
    const int nc = (int)(K / 256);  // blocks per row
    const int tid = threadIdx.x, lane = tid & 63, ks = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + F16_TM - 1) / F16_TM, (N + FM_TN - 1) / FM_TN, tmi, tni);
    const int64_t n0 = tni * FM_TN, m0 = tmi * F16_TM;
    const int c0 = (int)(blockIdx.y * bps), c1 = (int)((blockIdx.y + 1) * bps < nc ? (blockIdx.y + 1) * bps : nc);
    tile_row_flags<F16_TM, FM_THREADS>(bad, m0, M, nc, rowbad, anybad);

    // staging: 16-byte pieces P = tid and tid + 256 of each plane: row P / 32, piece j = P % 32 (halves 8j .. +7)
    // = step j / 4, k-slice j % 4, i.e. lane 16 (j % 4) + row of step j / 4, at slot fh_swz(lane, step) of the step;
    // threads < 16 one exponent
    const uint16_t *hsrc[2];
    int hslot[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int P = tid + 256 * i, r = P >> 5, j = P & 31;
        hsrc[i] = xh + (m0 + r < M ? m0 + r : M - 1) * K + 8 * j;
        hslot[i] = 64 * (j >> 2) + fh_swz(16 * (j & 3) + r, j >> 2);
    }
    const int64_t lo_off = xl - xh;  // the lo plane sits at the same offsets from xl
    const int64_t egm = m0 + (tid & 15) < M ? m0 + (tid & 15) : M - 1;
    v4i sa[4];
    int se = 0;
    auto fetch_a = [&](int b) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            sa[i] = *reinterpret_cast<const v4i *>(hsrc[i] + 256 * (int64_t)b);
            sa[2 + i] = *reinterpret_cast<const v4i *>(hsrc[i] + lo_off + 256 * (int64_t)b);
        }
        if (tid < F16_TM) se = ex[egm * nc + b];
    };
    auto put_a = [&](int buf) {
        uint8_t *st = lds + buf * FH_STAGE;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            reinterpret_cast<v4i *>(st)[hslot[i]] = sa[i];
            reinterpret_cast<v4i *>(st + FH_PLANE)[hslot[i]] = sa[2 + i];
        }
        if (tid < F16_TM) reinterpret_cast<int *>(st + 2 * FH_PLANE)[tid] = se;
    };

    int64_t wrow[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int nl = 32 * w + 16 * t + (lane & 15);
        wrow[t] = row0 + ((n0 + nl) < N ? (n0 + nl) : N - 1);
    }
    // two weight register sets used alternately (blocks b and b + 1), so a block's weights are requested during
    // the previous block without any copy of registers whose loads are still in flight (such a copy waits for every
    // outstanding load, the next block's staging included)
    Q6Regs wA[2], wB[2];
    auto fetch_w = [&](Q6Regs(&wr)[2], int b) {
#pragma unroll
        for (int t = 0; t < 2; t++) q6_load(wr[t], p, wrow[t], b, ks);
    };

    float accf[2][4];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) accf[t][v] = 0.0f;
    // every slice holds at least one chunk; the prefetches below are issued unconditionally (the last chunk's
    // re-read, when there is no next one), so the wait counts stay static and never fall back to waiting for
    // everything outstanding
    auto last = [&](int b) { return b < c1 ? b : c1 - 1; };
    fetch_a(c0);
    fetch_w(wA, c0);
    put_a(0);
    fetch_a(last(c0 + 1));
    __syncthreads();

    const v4f zero = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    auto chunk = [&](int b, const Q6Regs(&cw)[2]) {
        const uint8_t *st = lds + ((b - c0) & 1) * FH_STAGE;
        const v8h *ph = reinterpret_cast<const v8h *>(st), *pq = reinterpret_cast<const v8h *>(st + FH_PLANE);
        v4f acc[2] = {zero, zero};
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const v8h ah = ph[64 * s + fh_swz(lane, s)], al = pq[64 * s + fh_swz(lane, s)];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const v8h q = q6_codes(cw[t], s);
                // scale of this lane's 16-element group (2 s + ks / 2), as even part and low bit
                const uint32_t scw = s < 2 ? cw[t].sc.x : s < 4 ? cw[t].sc.y : s < 6 ? cw[t].sc.z : cw[t].sc.w;
                const int sc = (int)(int8_t)((scw >> (16 * (s & 1) + 8 * (ks >> 1))) & 0xFF);
                const _Float16 se2 = (_Float16)(float)(sc & ~1), so = (_Float16)(float)(sc & 1);
                const v8h q1 = q * se2, q2 = q * so;
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, q1, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, q1, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, q2, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, q2, acc[t], 0, 0, 0);
            }
        }
        if (b + 1 < c1) put_a((b + 1 - c0) & 1);
        fetch_a(last(b + 2));
        const int *exs = reinterpret_cast<const int *>(st + 2 * FH_PLANE);
        const int4 e4 = *reinterpret_cast<const int4 *>(exs + 4 * ks);
        const int ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const float dk = f16_to_f32((uint16_t)cw[t].d);
#pragma unroll
            for (int v = 0; v < 4; v++) accf[t][v] = accf[t][v] + ldexpf(dk * acc[t][v], ev[v]);
        }
        __syncthreads();
    };
    for (int b = c0; b < c1; b += 2) {
        fetch_w(wB, last(b + 1));
        chunk(b, wA);
        if (b + 1 >= c1) break;
        fetch_w(wA, last(b + 2));
        chunk(b + 1, wB);
    }

    float *dst = partial ? partial + (int64_t)blockIdx.y * M * N : c;
    const bool acc_c = ACC && partial == nullptr;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int64_t gn = n0 + 32 * w + 16 * t + (lane & 15);
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int mloc = 4 * ks + v;
            if (gn < N && rowbad[mloc] == 0) {
                float *o = dst + (m0 + mloc) * N + gn;
                *o = acc_c ? *o + accf[t][v] : accf[t][v];
            }
        }
    }
    if (!*anybad) return;
    for (int i = tid; i < F16_TM * FM_TN; i += FM_THREADS) {  // rows holding NaN/Inf: exact float dot products
        const int ml = i / FM_TN, nl = i % FM_TN;
        const int64_t gn2 = n0 + nl;
        if (rowbad[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = blockIdx.y == 0 ? exact_dot_row<kQ6K>(p, row0 + gn2, x + gm * K, K) : 0.0f;
        float *o = dst + gm * N + gn2;
        *o = acc_c ? *o + v : v;
    }
}

// out[m, i] = silu(g) * u with g, u the slice sums of partial rows i and I + i of activation row m, each added in
// slice order as fm_sum_kernel adds them: the same bits as fm_sum_kernel followed by swiglu_kernel.
__global__ void fm_sum_swiglu_kernel(const float *__restrict__ partial, float *__restrict__ out, int64_t M, int64_t I,
                                     int64_t ns) {
    const int64_t N = 2 * I, MN = M * N;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < M * I; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t m = t / I, i = t - m * I, og = m * N + i, ou = og + I;
        float g = partial[og], u = partial[ou];
        for (int64_t k = 1; k < ns; k += 4) {  // up to eight loads in flight, added in slice order
            float vg[4], vu[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                vg[q] = k + q < ns ? partial[(k + q) * MN + og] : 0.0f;
                vu[q] = k + q < ns ? partial[(k + q) * MN + ou] : 0.0f;
            }
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (k + q < ns) {
                    g = g + vg[q];
                    u = u + vu[q];
                }
        }
        out[t] = silu_ref(g) * u;
    }
}

}  // namespace

int launch_actq_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     int64_t M, bool acc, const int8_t *q, const float *d, const uint16_t *sj, const uint8_t *bad,
                     bool fast) {
    if (w->dtype != kQ4K) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq_mfma: q4_k only");
    // Row-tile height: 64 rows unless that leaves fewer than 160 workgroups (measured: 4096 x 14336 at M = 128
    // takes 74 us on 32-row tiles against 104 on 64; 14336 x 4096 at M = 128 or 512 is faster on 64).
    // trhip_set_launch_shape(TRHIP_KNOB_ACTQ_TM) overrides.
    const int64_t wgs64 = ((N + TN - 1) / TN) * ((M + 63) / 64);
    const int tm = ctx->force_actq_tm ? ctx->force_actq_tm : (wgs64 < 160 ? 32 : 64);
    // K slices (fast mode): two when K is long (at least 32 blocks) and the tiles fit on the CUs one workgroup each.
    // Measured (us, one slice -> two): 4096x14336 at M = 128 71.0 -> 52.0, at M = 512 121.5 -> 113.6; with 16
    // blocks (14336x4096 or 4096x4096 at M = 128) no gain; three or more slices were slower everywhere.
    // trhip_set_launch_shape(TRHIP_KNOB_ACTQ_TM, tm, S) overrides.
    int S = ctx->force_actq_slices;
    if (S == 0 && fast && w->nb >= 32) {
        const int64_t tiles = ((N + TN - 1) / TN) * ((M + tm - 1) / tm);
        S = tiles <= (ctx->sm_count > 0 ? ctx->sm_count : 256) ? 2 : 1;
    }
    if (tm == 32) return run_mfma<32>(ctx, w, row0, N, x, c, M, acc, q, d, sj, bad, fast, S);
    return run_mfma<64>(ctx, w, row0, N, x, c, M, acc, q, d, sj, bad, fast, S);
}

}  // namespace trhip

namespace trhip {

// Fast-mode M > 1 for q4_k and q6_k (tolerance): x as fixed-point planes (q4_k: int8 digits for fastm_mfma_q4k /
// fastm16_mfma_q4k; q6_k: two f16 planes for fastm16_q6k on 16-row tiles), the MFMA kernel over K slices, then the
// slices' sum in slice order.
int launch_gemm_rows_fast(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                          int64_t M, bool acc, float *swi) {
    const int dt = w->dtype;
    const int64_t K = w->K, nb = K / 256;
    if (dt != kQ4K && dt != kQ6K) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemm_rows_fast: q4_k and q6_k only");
    const bool t16 = dt != kQ4K || M <= F16_TM;  // 16-row tiles
    const int64_t tiles = ((N + FM_TN - 1) / FM_TN) * (t16 ? (M + F16_TM - 1) / F16_TM : (M + FM_TM - 1) / FM_TM);
    int64_t ns = (512 + tiles - 1) / tiles;  // K slices for about 512 workgroups
    if (ns > nb) ns = nb;
    const int64_t bps = (nb + ns - 1) / ns;
    ns = (nb + bps - 1) / bps;
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    const bool copy_x = reinterpret_cast<uintptr_t>(x) % 16 != 0;
    // q4_k: three int8 digit planes and the f16 msum parts; q6_k: two f16 planes
    const size_t xbytes = dt == kQ4K ? 3 * (size_t)(M * K) : 4 * (size_t)(M * K);
    const size_t o_dg = 0, o_ex = al(o_dg + xbytes), o_xs = al(o_ex + (size_t)(M * nb) * sizeof(int));
    const size_t o_bad = al(o_xs + (size_t)(M * nb) * 48), o_x = al(o_bad + (size_t)(M * nb));
    const size_t o_p = al(o_x + (copy_x ? (size_t)(M * K) * sizeof(float) : 0));
    const size_t total = o_p + (ns > 1 ? (size_t)(ns * M * N) * sizeof(float) : 0);
    int st = TRHIP_OK;
    uint8_t *ws = static_cast<uint8_t *>(workspace(ctx, total, &st));
    if (!ws) return st;
    const float *xa = x;
    if (copy_x) {
        hipError_t e = hipMemcpyAsync(ws + o_x, x, (size_t)(M * K) * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "gemm_rows_fast: align x");
        xa = reinterpret_cast<const float *>(ws + o_x);
    }
    uint8_t *bad = ws + o_bad;
    uint16_t *xh = reinterpret_cast<uint16_t *>(ws + o_dg), *xl = xh + M * K;
    if (dt == kQ4K)
        hipLaunchKernelGGL(digits_q4k_kernel, dim3((unsigned)((M * nb + 3) / 4)), dim3(256), 0, ctx->stream, xa, M, K,
                           reinterpret_cast<int8_t *>(ws + o_dg), reinterpret_cast<int *>(ws + o_ex),
                           reinterpret_cast<uint16_t *>(ws + o_xs), bad);
    else
        hipLaunchKernelGGL(halves_kernel, dim3((unsigned)((M * nb + 3) / 4)), dim3(256), 0, ctx->stream, xa, M, K, xh,
                           xl, reinterpret_cast<int *>(ws + o_ex), bad);
    if ((st = launch_check(ctx, dt == kQ4K ? "digits_q4k" : "halves")) != TRHIP_OK) return st;
    float *partial = ns > 1 ? reinterpret_cast<float *>(ws + o_p) : nullptr;
    dim3 grid((unsigned)tiles, (unsigned)ns), block(FM_THREADS);
    const int8_t *dg = reinterpret_cast<const int8_t *>(ws + o_dg);
    const int *ex = reinterpret_cast<const int *>(ws + o_ex);
    const uint16_t *xs = reinterpret_cast<const uint16_t *>(ws + o_xs);
    const bool acc_k = acc && !partial;
    const Planes pl = w->planes();
    if (dt == kQ6K) {
        if (acc_k)
            hipLaunchKernelGGL(fastm16_q6k<true>, grid, block, FH_LDS, ctx->stream, pl, N, row0, M, K, xa, xh, xl, ex,
                               bad, bps, c, partial);
        else
            hipLaunchKernelGGL(fastm16_q6k<false>, grid, block, FH_LDS, ctx->stream, pl, N, row0, M, K, xa, xh, xl, ex,
                               bad, bps, c, partial);
    } else if (t16) {  // LDS below 64 KB: no attribute needed
        if (acc_k)
            hipLaunchKernelGGL(fastm16_mfma_q4k<true>, grid, block, F16_LDS, ctx->stream, pl, N, row0, M, K, xa, dg, ex,
                               xs, bad, bps, c, partial);
        else
            hipLaunchKernelGGL(fastm16_mfma_q4k<false>, grid, block, F16_LDS, ctx->stream, pl, N, row0, M, K, xa, dg,
                               ex, xs, bad, bps, c, partial);
    } else {
        if (acc_k)
            hipLaunchKernelGGL(fastm_mfma_q4k<true>, grid, block, FM_LDS, ctx->stream, pl, N, row0, M, K, xa, dg, ex,
                               xs, bad, bps, c, partial);
        else
            hipLaunchKernelGGL(fastm_mfma_q4k<false>, grid, block, FM_LDS, ctx->stream, pl, N, row0, M, K, xa, dg, ex,
                               xs, bad, bps, c, partial);
    }
    if ((st = launch_check(ctx, "gemm_rows_fast")) != TRHIP_OK) return st;
    if (swi) {  // SwiGLU gate over [gate | up] = N = 2I columns, fused into the slice sum
        if (!partial) return launch_swiglu(ctx, c, M, N / 2, swi);
        const int64_t MI = M * (N / 2);
        const unsigned blocks = (unsigned)((MI + 255) / 256 < 4096 ? (MI + 255) / 256 : 4096);
        hipLaunchKernelGGL(fm_sum_swiglu_kernel, dim3(blocks), dim3(256), 0, ctx->stream, partial, swi, M, N / 2, ns);
        return launch_check(ctx, "fm_sum_swiglu");
    }
    if (!partial) return st;
    const int64_t MN = M * N;
    const unsigned blocks = (unsigned)((MN + 255) / 256 < 4096 ? (MN + 255) / 256 : 4096);
    if (acc)
        hipLaunchKernelGGL(fm_sum_kernel<true>, dim3(blocks), dim3(256), 0, ctx->stream, partial, c, MN, ns);
    else
        hipLaunchKernelGGL(fm_sum_kernel<false>, dim3(blocks), dim3(256), 0, ctx->stream, partial, c, MN, ns);
    return launch_check(ctx, "fm_sum");
}

}  // namespace trhip
