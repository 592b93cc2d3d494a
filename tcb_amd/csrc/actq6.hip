// actq6.hip -- act-quant prefill GEMM for q6_k weights on int8 matrix cores, bit-identical to dotQ6KQ8Go
// (tensor/cpu_quant_q8.go:378-407).
//
// Per 256-element block b and output (m, n) the reference computes, with the sub-block scales sc_j (signed bytes,
// 16 sub-blocks of 16 elements) and q6 codes in [0, 63]:
//   X = isum - 32 msum = sum_j sc_j sum_{i in j} (q6_i - 32) q8_i        exact in int32
//   t = fl(d fl(X));  acc = fl(acc + fl(t d8))                            blocks in order
// (isum - 32 msum regroups exactly: msum = sum_j sc_j bs_j and bs_j is the 16-sum of the q8 codes.)
//
// The sub-block sums T_j = sum_{i in j} (q6_i - 32) q8_i come from v_mfma_i32_16x16x64_i8 with the weights as the A
// operand. A row 4 r + s (weight row r of a group of four, slot s) holds row r's codes of sub-block 4 w + s in
// k-slice s and zeros in the other three slices, so the product's row 4 r + s is T_{4w+s} of weight row r. With the
// instruction's lane layout (lane l: A row / B column l % 16, k-slice l / 16 of 16 bytes; result register v of lane
// l: row 4 (l / 16) + v, column l % 16, checked on the device), lane l's four result registers are the four
// sub-block sums of (weight row l / 16 of the group, activation row l % 16 of the tile). The lane scales and adds
// them in int32 (v_mad_i32_i24, |sc T| < 2^23), X = sum over the block's four 64-element windows, then applies the
// reference's per-block epilogue. The codes q6 - 32 are signed bytes in [-32, 31], built from the repacked ql / qh
// planes; the masked A operand of a window is built once and serves every activation tile of the wave.
//
// Tiling: a workgroup is 8 waves over 128 weight rows (16 per wave: four groups of four) and 128 activation rows
// (eight 16-row tiles per wave). Per block, the activation codes (swizzled 16-byte pieces) and the weight rows'
// ql, qh and scale bytes move into LDS by buffer_load ... lds, double-buffered with one barrier per block; d and
// d8 go through LDS by plain loads. Activation rows holding NaN/Inf are computed with the exact fp32 dot.
#include "trhip_internal.hpp"
#include "mfma_util.hpp"

namespace trhip {
namespace {

constexpr int Q6_W = 8;                   // waves per workgroup
constexpr int Q6_TN = 16 * Q6_W;          // weight rows per workgroup
constexpr int Q6_THREADS = 64 * Q6_W;
template <int MT>                         // MT 16-row activation tiles per wave
struct Q6L {
    static constexpr int TM = 16 * MT;        // activation rows per workgroup
    static constexpr int ACT = TM * 256;      // activation codes of one block
    static constexpr int QL = Q6_TN * 128;    // ql bytes of the workgroup's weight rows
    static constexpr int QH = Q6_TN * 64;
    static constexpr int SC = Q6_TN * 16;
    static constexpr int DW = Q6_TN * 4;      // d of the weight rows, fp32
    static constexpr int D8 = TM * 4;         // d8 of the activation rows
    static constexpr int O_QL = ACT, O_QH = O_QL + QL, O_SC = O_QH + QH, O_DW = O_SC + SC, O_D8 = O_DW + DW;
    static constexpr int STAGE = O_D8 + D8;
    static constexpr size_t LDS = 2 * STAGE + (TM + 1) * sizeof(int);
};
static_assert(Q6L<8>::LDS <= 160 * 1024, "one workgroup per CU");

// Staging copies global memory into LDS with inline-asm buffer_load ... lds (dma16, trhip_internal.hpp): a copy the
// compiler sees makes it wait for every copy in flight before the block's first LDS read, and the next block's staging
// would never overlap the current block's MFMAs. The kernel waits for its copies itself before each block's barrier.
__device__ __forceinline__ void q6_dma16(dma_rsrc r, uint32_t voffset, uint32_t soffset, void *l) {
    dma16(r, lds_addr(l), voffset, soffset);
}

// Activation piece (row, 16-byte column c) sits at slot 16 row + (c ^ (row & 7)): the eight rows a quarter-wave
// reads in one pass fall on distinct banks.
__device__ __forceinline__ int q6_act_slot(int row, int c) { return 16 * row + (c ^ (row & 7)); }

// Signed codes q6 - 32 of four elements: low (K2 = 0) or high nibbles of the ql dword L, with the qh dword H's bit
// pairs at shift 2 k (k = 2 K2 + kb), as bytes. q + 96 never carries out of a byte; xor 128 then gives q - 32.
template <int K>
__device__ __forceinline__ uint32_t q6_codes(uint32_t L, uint32_t H) {
    const uint32_t lo = K < 2 ? (L & 0x0F0F0F0Fu) : ((L >> 4) & 0x0F0F0F0Fu);
    const uint32_t hi = K == 0 ? ((H << 4) & 0x30303030u)
                      : K == 1 ? ((H << 2) & 0x30303030u)
                      : K == 2 ? (H & 0x30303030u)
                               : ((H >> 2) & 0x30303030u);
    return ((lo | hi) + 0x60606060u) ^ 0x80808080u;
}

template <bool ACC, int MT>
__global__ __launch_bounds__(Q6_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void actq6_mfma(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const int8_t *__restrict__ q, const float *__restrict__ d8g, const uint8_t *__restrict__ bad_blk,
    float *__restrict__ c) {
    using L = Q6L<MT>;
    constexpr int Q6_TM = L::TM, Q6_MT = MT;
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowstate = reinterpret_cast<int *>(lds + 2 * L::STAGE);  // [TM] 0 ok, 1 NaN/Inf row, 2 outside M
    int *anybad = rowstate + Q6_TM;

    const int nb = (int)p.nb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + Q6_TM - 1) / Q6_TM, (N + Q6_TN - 1) / Q6_TN, tmi, tni);
    const int64_t n0 = tni * Q6_TN, m0 = tmi * Q6_TM;
    tile_row_flags<Q6_TM, Q6_THREADS>(bad_blk, m0, M, nb, rowstate, anybad);

    // buffers with 32-bit offsets (the launcher checks they fit); reads past the end return 0
    const dma_rsrc rq = dma_desc(q, (uint32_t)(M * K));
    const dma_rsrc rql = dma_desc(p.qs, (uint32_t)((row0 + N) * nb * 128));
    const dma_rsrc rqh = dma_desc(p.aux, (uint32_t)((row0 + N) * nb * 64));
    const dma_rsrc rsc = dma_desc(p.sc, (uint32_t)((row0 + N) * nb * 16));
    const int64_t wr0 = row0 + n0;  // the workgroup's first store row

    // DMA offsets. Activation instruction j (TM / 4 per block, TM / 32 per wave): rows 4 j .. 4 j + 3, lane L -> row
    // 4 j + L / 16, column (L % 16) ^ (row & 7). Weight ql instruction j (16 per block, two per wave): rows
    // 8 j .. +7, lane L -> row 8 j + L / 8, piece L % 8. qh (8, one per wave): rows 16 j + L / 4, piece L % 4. sc
    // (2, waves 0 and 1): row 64 j + L.
    constexpr int AI = Q6_TM / 32;  // activation instructions per wave
    uint32_t va[AI];
#pragma unroll
    for (int i = 0; i < AI; i++) {
        const int j = AI * w + i, row = 4 * j + (lane >> 4), col = (lane & 15) ^ (row & 7);
        va[i] = (uint32_t)((m0 + row) * K + 16 * col);
    }
    uint32_t vql[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int j = 2 * w + i, row = 8 * j + (lane >> 3);
        vql[i] = (uint32_t)((wr0 + row) * nb * 128 + 16 * (lane & 7));
    }
    const uint32_t vqh = (uint32_t)((wr0 + 16 * w + (lane >> 2)) * nb * 64 + 16 * (lane & 3));
    const uint32_t vsc = (uint32_t)((wr0 + 64 * (w & 1) + lane) * nb * 16);
    // d of weight row tid (threads < TN) and d8 of activation row tid - TN (TN <= tid < TN + TM), plain loads
    const int64_t drow = wr0 + tid < row0 + N ? wr0 + tid : row0 + N - 1;
    const int64_t d8row = m0 + (tid - Q6_TN) < M ? m0 + (tid - Q6_TN) : M - 1;

    auto stage = [&](int b, int buf) {
        uint8_t *sb = lds + buf * L::STAGE;
#pragma unroll
        for (int i = 0; i < AI; i++) q6_dma16(rq, va[i], (uint32_t)(256 * b), sb + 1024 * (AI * w + i));
#pragma unroll
        for (int i = 0; i < 2; i++) q6_dma16(rql, vql[i], (uint32_t)(128 * b), sb + L::O_QL + 1024 * (2 * w + i));
        q6_dma16(rqh, vqh, (uint32_t)(64 * b), sb + L::O_QH + 1024 * w);
        if (w < 2) q6_dma16(rsc, vsc, (uint32_t)(16 * b), sb + L::O_SC + 1024 * w);
    };
    float dnext = 0.0f;
    auto fetch_scales = [&](int b) {
        if (tid < Q6_TN) dnext = f16_to_f32(p.d[drow * nb + b]);
        else if (tid < Q6_TN + Q6_TM) dnext = d8g[d8row * nb + b];
    };
    auto put_scales = [&](int buf) {
        uint8_t *sb = lds + buf * L::STAGE;
        if (tid < Q6_TN) reinterpret_cast<float *>(sb + L::O_DW)[tid] = dnext;
        else if (tid < Q6_TN + Q6_TM) reinterpret_cast<float *>(sb + L::O_D8)[tid - Q6_TN] = dnext;
    };

    // lane roles: as A (weights) row i = lane % 16 of group g4: weight row 16 w + 4 g4 + i / 4, slot i % 4; k-slice
    // kg = lane / 16; valid (non-zero) only where slot == kg. As a result: weight row 16 w + 4 g4 + lane / 16,
    // activation row 16 t + lane % 16.
    const int ai = lane & 15, kg = lane >> 4;
    const uint32_t amask = (ai & 3) == kg ? 0xFFFFFFFFu : 0u;
    // sub-block 4 win + kg of the A row: ql dwords 8 t0 + cc, +1, 8 t0 + 8 + cc, +1 and qh dwords 4 t0 + 2 n2, +1,
    // 4 t0 + 4 + 2 n2, +1, with n2 = win / 2, t0 = 2 (kg & 1), cc = 4 n2 + 2 (kg / 2); windows 2 n2 and 2 n2 + 1 share
    // them (low / high nibbles, qh bit pairs 2 k with k = 2 (win & 1) + kg / 2)
    const int t0 = 2 * (kg & 1), kb = kg >> 1;

    float acc[4][Q6_MT];
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++)
#pragma unroll
        for (int t = 0; t < Q6_MT; t++) acc[g4][t] = 0.0f;

    fetch_scales(0);
    stage(0, 0);
    put_scales(0);
    for (int b = 0; b < nb; b++) {
        // block b (DMA and scales) is in stage b & 1 once every load has landed; after the barrier nobody reads
        // the other stage (block b - 1) any more
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (b + 1 < nb) {
            fetch_scales(b + 1);
            stage(b + 1, (b + 1) & 1);
        }
        const uint8_t *sb = lds + (b & 1) * L::STAGE;
        int X[4][Q6_MT];
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++)
#pragma unroll
            for (int t = 0; t < Q6_MT; t++) X[g4][t] = 0;
#pragma unroll 1
        for (int win = 0; win < 4; win++) {
            // this lane's A row (weight row 16 w + 4 g4 + ai / 4, sub-block 4 win + kg) for the four groups, and the
            // scales sc_{4 win + v} of the result role's weight row 16 w + 4 g4 + kg
            const int n2 = win >> 1, hw = win & 1, cc = 4 * n2 + 2 * kb;
            v4i A[4];
            int sd[4];
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int r = 16 * w + 4 * g4 + (ai >> 2);
                const uint32_t *ql = reinterpret_cast<const uint32_t *>(sb + L::O_QL + 128 * r);
                const uint32_t *qh = reinterpret_cast<const uint32_t *>(sb + L::O_QH + 64 * r);
                const uint2 l0 = *reinterpret_cast<const uint2 *>(ql + 8 * t0 + cc);
                const uint2 l1 = *reinterpret_cast<const uint2 *>(ql + 8 * t0 + 8 + cc);
                const uint2 h0 = *reinterpret_cast<const uint2 *>(qh + 4 * t0 + 2 * n2);
                const uint2 h1 = *reinterpret_cast<const uint2 *>(qh + 4 * t0 + 4 + 2 * n2);
                const uint32_t Lw[4] = {l0.x, l0.y, l1.x, l1.y}, Hw[4] = {h0.x, h0.y, h1.x, h1.y};
                uint32_t cw[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // k = 2 hw + kb: low nibbles for windows 0 and 2, high for 1 and 3
                    if (hw == 0) cw[e] = kb ? q6_codes<1>(Lw[e], Hw[e]) : q6_codes<0>(Lw[e], Hw[e]);
                    else cw[e] = kb ? q6_codes<3>(Lw[e], Hw[e]) : q6_codes<2>(Lw[e], Hw[e]);
                }
                A[g4] = (v4i){(int)(cw[0] & amask), (int)(cw[1] & amask), (int)(cw[2] & amask), (int)(cw[3] & amask)};
                sd[g4] = reinterpret_cast<const int *>(sb + L::O_SC + 16 * (16 * w + 4 * g4 + kg))[win];
            }
#pragma unroll
            for (int t = 0; t < Q6_MT; t++) {
                const v4i B = *reinterpret_cast<const v4i *>(sb + 16 * q6_act_slot(16 * t + ai, 4 * win + kg));
                v4i D[4];
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++)
                    D[g4] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[g4], B, (v4i){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++)
#pragma unroll
                    for (int v = 0; v < 4; v++)  // signed-byte scale times a 24-bit sum: v_mul_i32_i24
                        X[g4][t] += ((sd[g4] << (24 - 8 * v)) >> 24) * ((D[g4][v] << 8) >> 8);
            }
        }
        // per-block epilogue in the reference's rounding order
        const float *dws = reinterpret_cast<const float *>(sb + L::O_DW);
        const float *d8s = reinterpret_cast<const float *>(sb + L::O_D8);
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            const float dd = dws[16 * w + 4 * g4 + kg];
#pragma unroll
            for (int t = 0; t < Q6_MT; t++) {
                const float tt = dd * (float)X[g4][t];
                acc[g4][t] = acc[g4][t] + tt * d8s[16 * t + ai];
            }
        }
        // the next block's scales into the other stage (last read before this block's barrier); the next barrier
        // publishes them
        if (b + 1 < nb) put_scales((b + 1) & 1);
    }

#pragma unroll
    for (int g4 = 0; g4 < 4; g4++) {
        const int64_t gn = n0 + 16 * w + 4 * g4 + kg;
#pragma unroll
        for (int t = 0; t < Q6_MT; t++) {
            const int ml = 16 * t + ai;
            if (gn < N && rowstate[ml] == 0) {
                float *o = c + (m0 + ml) * N + gn;
                *o = ACC ? *o + acc[g4][t] : acc[g4][t];
            }
        }
    }
    // rows holding NaN/Inf take the exact fp32 path (quantGemv) on their own; rare
    if (!*anybad) return;
    for (int i = tid; i < Q6_TM * Q6_TN; i += Q6_THREADS) {
        const int ml = i / Q6_TN, nl = i % Q6_TN;
        const int64_t gn2 = n0 + nl;
        if (rowstate[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = exact_dot_row<kQ6K>(p, row0 + gn2, x + gm * K, K);
        float *o = c + gm * N + gn2;
        *o = ACC ? *o + v : v;
    }
}

}  // namespace

// Taken for q6_k act-quant with at least 8 activation rows when every buffer offset fits 32 bits.
bool actq6_mfma_applies(int64_t M, int64_t N, int64_t row0, int64_t K) {
    const int64_t nb = K / 256;
    return M >= 8 && M * K < ((int64_t)1 << 32) && (row0 + N + Q6_TN) * nb * 128 < ((int64_t)1 << 32);
}

int launch_actq6_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                      int64_t M, bool acc, const int8_t *q, const float *d, const uint8_t *bad) {
    if (w->dtype != kQ6K) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq6_mfma: q6_k only");
    if (!actq6_mfma_applies(M, N, row0, w->K)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq6_mfma: shape");
    // 128 activation rows per workgroup, or 64 where 128 would leave CUs without a workgroup
    const int cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
    const int64_t nt = (N + Q6_TN - 1) / Q6_TN;
    const bool small = ((M + 127) / 128) * nt < cus;
    auto go = [&](auto kern, int64_t tm, size_t lds) {
        const int64_t wgs = ((M + tm - 1) / tm) * nt;
        if (wgs >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq6_mfma: grid too large");
        int st = allow_dyn_lds(ctx, reinterpret_cast<const void *>(kern), lds, "actq6_mfma: LDS size");
        if (st != TRHIP_OK) return st;
        hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(Q6_THREADS), lds, ctx->stream, w->planes(), N, row0, M,
                           w->K, x, q, d, bad, c);
        return launch_check(ctx, "actq6_mfma");
    };
    if (small) return acc ? go(&actq6_mfma<true, 4>, 64, Q6L<4>::LDS) : go(&actq6_mfma<false, 4>, 64, Q6L<4>::LDS);
    return acc ? go(&actq6_mfma<true, 8>, 128, Q6L<8>::LDS) : go(&actq6_mfma<false, 8>, 128, Q6L<8>::LDS);
}

}  // namespace trhip
