// actq4.hip -- act-quant prefill GEMM for q4_0 weights on int8 matrix cores, bit-identical to dotQ4Q8Go
// (tensor/cpu_quant_q8.go:74-87).
//
// Per 32-element block b and output (m, n) the reference computes
//   isum = sum_i (q4_i - 8) q8_i            exact in int32 (|isum| <= 32 * 8 * 127)
//   t = fl(d_w d8);  acc = fl(acc + fl(t fl(isum)))        blocks in order
// One block is exactly the K of v_mfma_i32_32x32x32_i8: the activation codes are the A operand (32 rows), the weight
// codes q4 - 8 (signed bytes) the B operand (32 columns). Lane l of a block's B operand holds elements
// 16 (l / 32) .. +15 of weight row l % 32, i.e. the low (l < 32) or high (l >= 32) nibbles of the block's 16 bytes
// (byte j holds elements j and j + 16, tensor/quant.go:149-155); lane l of the A operand the same elements of
// activation row l % 32. The result's lane l holds rows 8 j + 4 (l / 32) + r (j, r < 4) of column l % 32 (the
// layout the 32x32 int8 products of the other matrix-core kernels use), so each lane owns sixteen outputs of one
// weight row. The scale products t of a block's 64 x 32 outputs come from the matrix cores too (a two-block
// 32x32x1 fp32 product of the d8 column and the d_w row, in the same layout), which leaves the VALU three
// instructions per output and block (convert, multiply, add: the reference's rounding steps, unfused); the VALU is
// what bounds this kernel, so the products of block b + 1 are issued before block b is folded in.
//
// Tiling: a workgroup is 4 waves over 128 weight rows (32 per wave) and 64 activation rows (two 32-row tiles).
// Eight blocks (256 elements) form one LDS stage: the activation and weight codes in swizzled 16-byte pieces, the
// activation scales d8 transposed to [block][row] and the weight scales as fp16, all moved by buffer_load ... lds,
// double-buffered with one barrier per stage. Activation rows holding NaN/Inf are computed with the exact fp32 dot.
#include "trhip_internal.hpp"
#include "mfma_util.hpp"

namespace trhip {
namespace {

constexpr int Q4A_W = 4;                 // waves per workgroup
constexpr int Q4A_TN = 32 * Q4A_W;       // weight rows per workgroup
constexpr int Q4A_MT = 2;                // 32-row activation tiles per wave
constexpr int Q4A_TM = 32 * Q4A_MT;      // activation rows per workgroup
constexpr int Q4A_THREADS = 64 * Q4A_W;
constexpr int Q4A_BPS = 8;               // blocks per stage
struct Q4AL {
    static constexpr int ACT = Q4A_TM * 32 * Q4A_BPS;   // activation codes of a stage
    static constexpr int W = Q4A_TN * 16 * Q4A_BPS;     // weight codes
    static constexpr int D8 = Q4A_TM * 4 * Q4A_BPS;     // d8 as [block][row]
    static constexpr int DW = Q4A_TN * 2 * Q4A_BPS;     // weight scales as [row][block] fp16
    static constexpr int O_W = ACT, O_D8 = O_W + W, O_DW = O_D8 + D8;
    static constexpr int STAGE = O_DW + DW;
    static constexpr size_t LDS = 2 * STAGE + (Q4A_TM + 1) * sizeof(int);
};
static_assert(Q4AL::LDS <= 80 * 1024, "two workgroups per CU");

// Staging copies global memory into LDS with inline-asm buffer_load ... lds (dma16 / dma4, trhip_internal.hpp): a copy
// the compiler sees makes it wait for every copy in flight before the stage's first LDS read, and the next stage would
// never overlap the current one's MFMAs. The kernel waits for its copies itself before each stage's barrier.
__device__ __forceinline__ void q4a_dma16(dma_rsrc r, uint32_t voffset, uint32_t soffset, void *l) {
    dma16(r, lds_addr(l), voffset, soffset);
}
__device__ __forceinline__ void q4a_dma4(dma_rsrc r, uint32_t voffset, uint32_t soffset, void *l) {
    dma4(r, lds_addr(l), voffset, soffset);
}

// Activation piece (row, 16-byte column c of the stage's 256 bytes) at slot 16 row + (c ^ (row & 15)); weight piece
// (row, block bb) at slot 8 row + (bb ^ (row & 7)): the rows a quarter-wave reads in one pass fall on distinct
// banks.
__device__ __forceinline__ int q4a_act_slot(int row, int c) { return 16 * row + (c ^ (row & 15)); }
__device__ __forceinline__ int q4a_w_slot(int row, int bb) { return 8 * row + (bb ^ (row & 7)); }

// (two waves per SIMD, which the LDS allows anyway: with the register budget of that occupancy the products stay in
// VGPRs, and the epilogue reads them without a copy out of the accumulator registers)
template <bool ACC>
__global__ __launch_bounds__(Q4A_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void actq4_mfma(const Planes p, int64_t N, int64_t row0, int64_t M,
                                                          int64_t K, const float *__restrict__ x,
                                                          const int8_t *__restrict__ q, const float *__restrict__ d8g,
                                                          const uint8_t *__restrict__ bad_blk, float *__restrict__ c) {
    using L = Q4AL;
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowstate = reinterpret_cast<int *>(lds + 2 * L::STAGE);  // [TM] 0 ok, 1 NaN/Inf row, 2 outside M
    int *anybad = rowstate + Q4A_TM;

    const int nb = (int)p.nb, ns = nb / Q4A_BPS;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + Q4A_TM - 1) / Q4A_TM, (N + Q4A_TN - 1) / Q4A_TN, tmi, tni);
    const int64_t n0 = tni * Q4A_TN, m0 = tmi * Q4A_TM;
    tile_row_flags<Q4A_TM, Q4A_THREADS>(bad_blk, m0, M, nb, rowstate, anybad);

    // buffers with 32-bit offsets (the launcher checks they fit); reads past the end return 0
    const dma_rsrc rq = dma_desc(q, (uint32_t)(M * K));
    const dma_rsrc rw = dma_desc(p.qs, (uint32_t)((row0 + N) * nb * 16));
    const dma_rsrc rd8 = dma_desc(d8g, (uint32_t)(M * nb * 4));
    const dma_rsrc rdw = dma_desc(p.d, (uint32_t)((row0 + N) * nb * 2));
    const int64_t wr0 = row0 + n0;

    // DMA offsets per stage s (soffset adds the stage's position). Activation instruction j (16 per stage, four
    // per wave): rows 4 j .. +3, lane L -> row 4 j + L / 16, slot column L % 16 = column ^ (row & 15). Weight
    // instruction j (16, four per wave): rows 8 j .. +7, lane L -> row 8 j + L / 8, slot L % 8 = block ^ (row & 7).
    // d8 (8 instructions of 4 bytes, two per wave): instruction j = block j of the stage, lane L = row L. Weight
    // scales (two instructions of 16 bytes, waves 0 and 1): lane L -> row 64 w + L, the stage's 8 fp16 values.
    uint32_t va[4], vw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int j = 4 * w + i;
        const int ar = 4 * j + (lane >> 4), ac = (lane & 15) ^ (ar & 15);
        va[i] = (uint32_t)((m0 + ar) * K + 16 * ac);
        const int wrw = 8 * j + (lane >> 3), wb = (lane & 7) ^ (wrw & 7);
        vw[i] = (uint32_t)((wr0 + wrw) * nb * 16 + 16 * wb);
    }
    const uint32_t vd8 = (uint32_t)((m0 + lane) * nb * 4);
    const uint32_t vdw = (uint32_t)((wr0 + 64 * (w & 1) + lane) * nb * 2);

    auto stage = [&](int s, int buf) {
        uint8_t *sb = lds + buf * L::STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) q4a_dma16(rq, va[i], (uint32_t)(256 * s), sb + 1024 * (4 * w + i));
#pragma unroll
        for (int i = 0; i < 4; i++) q4a_dma16(rw, vw[i], (uint32_t)(128 * s), sb + L::O_W + 1024 * (4 * w + i));
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int j = 2 * w + i;
            q4a_dma4(rd8, vd8, (uint32_t)(4 * (Q4A_BPS * s + j)), sb + L::O_D8 + 256 * j);
        }
        if (w < 2) q4a_dma16(rdw, vdw, (uint32_t)(16 * s), sb + L::O_DW + 1024 * w);
    };

    // lane roles: B (weights) column n = lane % 32 of this wave's 32 rows, elements 16 h .. +15 of the block
    // (h = lane / 32: low or high nibbles); A (activations) row lane % 32 of a tile, the same elements; result:
    // weight row 32 w + lane % 32, activation rows 8 j + 4 h + r of the tile
    const int nl = lane & 31, h = lane >> 5;
    const int wrow = 32 * w + nl;
    const int nsh = 4 * h;  // low nibbles for the lanes of k-slice 0, high for slice 1

    float acc[Q4A_MT][16];
#pragma unroll
    for (int t = 0; t < Q4A_MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[t][v] = 0.0f;

    // One block's products: C[t] = the int8 sums of activation tile t (32x32x32 i8), T = t = fl(d_w d8) for both
    // tiles as the two-block 32x32x1 fp32 product (block t = tile t: lane l gives A = d8 of activation row l of the
    // 64, B = d_w of weight row l % 32; D = a b + 0, one rounding, registers 16 t .. +15 in the int8 product's
    // layout).
    auto products = [&](const uint8_t *sb, int bb, v16i (&C)[Q4A_MT], v32f &T) {
        const uint4 raw = *reinterpret_cast<const uint4 *>(sb + L::O_W + 16 * q4a_w_slot(wrow, bb));
        const uint32_t rw4[4] = {raw.x, raw.y, raw.z, raw.w};
        v4i B;
#pragma unroll
        for (int e = 0; e < 4; e++)  // q4 - 8 as bytes: q + 120 never carries out of a byte, xor 128
            B[e] = (int)((((rw4[e] >> nsh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u);
        const float d8 = reinterpret_cast<const float *>(sb + L::O_D8)[Q4A_TM * bb + lane];
        const float dw = f16_to_f32(reinterpret_cast<const uint16_t *>(sb + L::O_DW)[Q4A_BPS * wrow + bb]);
        T = __builtin_amdgcn_mfma_f32_32x32x1f32(d8, dw, (v32f){0.0f}, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < Q4A_MT; t++) {
            const v4i A = *reinterpret_cast<const v4i *>(sb + 16 * q4a_act_slot(32 * t + nl, 2 * bb + h));
            C[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, (v16i){0}, 0, 0, 0);
        }
    };

    stage(0, 0);
    for (int s = 0; s < ns; s++) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // stage s has landed (this wave's copies, then everyone's at the barrier); nobody reads the other
        if (s + 1 < ns) stage(s + 1, (s + 1) & 1);
        const uint8_t *sb = lds + (s & 1) * L::STAGE;
        // software-pipelined over the stage's blocks: block bb + 1's products are in flight on the matrix cores
        // while the VALU folds block bb's into the sums
        v16i C[Q4A_MT];
        v32f T;
        products(sb, 0, C, T);
#pragma unroll
        for (int bb = 0; bb < Q4A_BPS; bb++) {
            v16i Cn[Q4A_MT];
            v32f Tn;
            if (bb + 1 < Q4A_BPS) products(sb, bb + 1, Cn, Tn);
#pragma unroll
            for (int t = 0; t < Q4A_MT; t++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[t][v] = acc[t][v] + T[16 * t + v] * (float)C[t][v];
            if (bb + 1 < Q4A_BPS) {
#pragma unroll
                for (int t = 0; t < Q4A_MT; t++) C[t] = Cn[t];
                T = Tn;
            }
        }
    }

    const int64_t gn = n0 + wrow;
#pragma unroll
    for (int t = 0; t < Q4A_MT; t++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int ml = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
            if (gn < N && rowstate[ml] == 0) {
                float *o = c + (m0 + ml) * N + gn;
                *o = ACC ? *o + acc[t][v] : acc[t][v];
            }
        }
    }
    // rows holding NaN/Inf take the exact fp32 path (quantGemv) on their own; rare
    if (!*anybad) return;
    for (int i = tid; i < Q4A_TM * Q4A_TN; i += Q4A_THREADS) {
        const int ml = i / Q4A_TN, nl2 = i % Q4A_TN;
        const int64_t gn2 = n0 + nl2;
        if (rowstate[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = exact_dot_row<kQ4>(p, row0 + gn2, x + gm * K, K);
        float *o = c + gm * N + gn2;
        *o = ACC ? *o + v : v;
    }
}

}  // namespace

// Taken for q4_0 act-quant with at least 8 activation rows, a block count that is a multiple of the stage's 8 and
// every buffer offset within 32 bits.
bool actq4_mfma_applies(int64_t M, int64_t N, int64_t row0, int64_t K) {
    const int64_t nb = K / 32;
    return M >= 8 && nb % Q4A_BPS == 0 && M * K < ((int64_t)1 << 32) &&
           (row0 + N + Q4A_TN) * nb * 16 < ((int64_t)1 << 32);
}

int launch_actq4_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                      int64_t M, bool acc, const int8_t *q, const float *d, const uint8_t *bad) {
    if (w->dtype != kQ4) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq4_mfma: q4_0 only");
    if (!actq4_mfma_applies(M, N, row0, w->K)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq4_mfma: shape");
    const int64_t wgs = ((M + Q4A_TM - 1) / Q4A_TM) * ((N + Q4A_TN - 1) / Q4A_TN);
    if (wgs >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "actq4_mfma: grid too large");
    auto go = [&](auto kern) {
        int st = allow_dyn_lds(ctx, reinterpret_cast<const void *>(kern), Q4AL::LDS, "actq4_mfma: LDS size");
        if (st != TRHIP_OK) return st;
        hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(Q4A_THREADS), Q4AL::LDS, ctx->stream, w->planes(), N, row0,
                           M, w->K, x, q, d, bad, c);
        return launch_check(ctx, "actq4_mfma");
    };
    return acc ? go(&actq4_mfma<true>) : go(&actq4_mfma<false>);
}

}  // namespace trhip
