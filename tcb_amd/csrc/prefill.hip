// prefill.hip -- act-quant prefill GEMM for q4_k (and, below, q6_k) weights on int8 MFMA, 128 activation rows x 32
// weight rows per wave, bit-identical to tensor/cpu_quant_q8.go:91-116 (dotQ4KQ8Go) like actq_mfma_q4k, and to
// :378-407 (dotQ6KQ8Go) for q6_k. Taken for grids large enough to fill the device (at least 192 workgroups of
// 128 x 256).
//
// Arithmetic (same as actq_mfma_q4k): per block b and output (m, n), with sc_j = 8 s1 + s0,
//   isum = sum_i (s0 q4)_i q8_i + 8 sum_i (s1 q4)_i q8_i      two v_mfma_i32_32x32x32_i8 accumulations, exact
//   msum = sum_j S_j m_j, S_j = 64 Sh_j + Sl_j                 one v_mfma_f32_32x32x16_f16, exact
//   t = fl(fl(d fl(isum)) - fl(dmin fl(msum)));  acc = fl(acc + fl(t d8))   blocks in order
//
// Why this shape. Measured on the device (trhip_mfma_probe and kernels of the same structure): int8 MFMA issues
// every ~34 cycle units at two waves per SIMD, and independent VALU work hides under it when it is issued between
// the MFMAs of the same wave (seven VALU per MFMA: ~42 units). A VALU burst after a tile's MFMAs does not hide, and
// VALU that reads a tile's sums right after its last MFMA stalls the wave for the MFMA latency. The exact epilogue
// costs seven VALU per output and block, i.e. seven per MFMA of a 32x32 tile. So:
//   - each wave expands its 32 weight rows' block once (both planes of all eight sub-blocks, 64 registers) and runs
//     four 32-row activation tiles through it: the expansion's ~135 VALU are spread over 68 MFMAs;
//   - two accumulator sets are used in turn: while tile t's 16 MFMAs run into one set, the epilogue of tile t - 1
//     (the previous block's last tile for t = 0) reads the other, two outputs after each MFMA pair;
//   - weights go to LDS with the activations (global_load_lds, no registers), leaving the registers for the above:
//     eight waves (256 weight rows) per workgroup, one workgroup per CU, two stages.
//
// Staging: the quantizer writes codes, msum operands and scales in the tiled layout (trhip_internal.hpp), so a
// block's activation data is 9 KB per 32-row tile of 1 KB pieces in operand order, each moved by one
// global_load_lds_dwordx4; each wave moves its own weight rows' header and codes the same way. One barrier per
// block: block b + 1 is in flight while block b is computed.
#include "trhip_internal.hpp"
#include "mfma_util.hpp"

namespace trhip {
namespace {

constexpr int PF_W = 8;                 // waves per workgroup, each owning 32 weight rows
constexpr int PF_TN = 32 * PF_W;        // weight rows per workgroup
constexpr int PF_THREADS = 64 * PF_W;
constexpr int PF_MT = 4;                // 32-row activation tiles per wave
struct Pf {
    static constexpr int TM = 32 * PF_MT;                   // activation rows per workgroup (and per wave)
    static constexpr int A = PF_MT * 8192, S = PF_MT * 1024; // codes, msum operands of one block
    static constexpr int WREG = 512 + 4096;                 // one wave's weight rows: 32 headers, then 32 x 128 codes
    static constexpr int STAGE = A + S + PF_W * WREG;
    static constexpr int D = PF_MT * 128;                   // d8 of one block (slot b % 3, read one block later)
    static constexpr int DOFF = 2 * STAGE;
    static constexpr size_t LDS = DOFF + 3 * D + (TM + 1) * sizeof(int);
    static constexpr int PIECES = 9 * PF_MT;                // 1 KB activation pieces per stage
};
static_assert(Pf::LDS <= 160 * 1024, "one workgroup per CU");

// The staging copies global memory into LDS with buffer_load ... lds (dma16 / dma4, trhip_internal.hpp), issued as
// inline assembly: seen by the compiler, such a copy makes it wait for every copy in flight before the block's first
// LDS read, so the next block's staging would never overlap the current block's work. The kernel waits for its copies
// itself, once per block, before the barrier.

// Epilogue kinds: q4_k in the reference's rounding order, q4_k fast, q6_k (exact).
enum { PF_Q4K = 0, PF_Q4K_FAST = 1, PF_Q6K = 2 };

// The per-block epilogue of one output. q4_k (isum = p0 + 8 p1): exact, in the reference's rounding order (seven
// VALU), or fast, the same integer sums with the two products and the accumulation fused (five VALU; within 1e-4 of
// the exact result). q6_k (X = p0 + 128 p1, tensor/cpu_quant_q8.go:404-405): t = fl(d fl(X)), acc = fl(acc + fl(t d8))
// (five VALU); cm and dm are not used.
template <int EK>
__device__ __forceinline__ float pf_epilogue(float acc, int p0, int p1, float cm, float dd, float dm, float d8) {
    if (EK == PF_Q6K) {
        const float tt = dd * (float)(p0 + 128 * p1);
        return acc + tt * d8;
    }
    const int isum = p0 + 8 * p1;
    if (EK == PF_Q4K_FAST) return fmaf(fmaf(-dm, cm, dd * (float)isum), d8, acc);
    const float tt = (dd * (float)isum) - (dm * cm);
    return acc + tt * d8;
}

// Eight integers below 64 (the bytes of lo, then hi) times c (1 or 64) as f16: v_perm_b32 places each byte under
// 0x64, giving the f16 value 1024 + v; subtracting 1024 and multiplying by c are both exact (v c <= 4032). (A fused
// (1024 + v) c - 1024 c is not usable: -1024 * 64 is beyond the f16 range.)
__device__ __forceinline__ v8h small_f16x8(uint32_t lo, uint32_t hi, _Float16 c) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 cc = (h2){c, c}, off = (h2){(_Float16)(-1024.0f), (_Float16)(-1024.0f)};
    auto pair = [&](uint32_t v, uint32_t sel) {
        const h2 x = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, v, sel));
        return __builtin_bit_cast(uint32_t, (x + off) * cc);
    };
    return __builtin_bit_cast(v8h, make_uint4(pair(lo, 0x04010400u), pair(lo, 0x04030402u), pair(hi, 0x04010400u),
                                              pair(hi, 0x04030402u)));
}

// One 32-row tile of a block: 16 int8 MFMAs into (c0, c1), and between them the epilogue of the pending tile held in
// (p0, p1) with msum pcm, the pending block's d, dmin and the d8 of its rows (pd8, this lane's rows at + 8 (v / 4)
// + (v % 4)). The pending sums are final only once the previous tile's last MFMAs have completed, so the first MFMA
// pair runs alone and the sixteen outputs follow the next seven pairs (two each, four after the last).
template <int EK>
__device__ __forceinline__ void pf_tile(v16i &c0, v16i &c1, const v16i &p0, const v16i &p1, const v16f &pcm, float pdd,
                                        float pdm, float *pacc, const float *pd8, const v4i *ar, const v4i (&b0)[8],
                                        const v4i (&b1)[8]) {
    c0 = (v16i){0};
    c1 = (v16i){0};
    // LDS reads complete in order, so each is issued a step before it is used and after everything used earlier:
    // step kc issues the d8 of step kc + 1, then A of step kc + 2
    v4i a[3];
    a[0] = ar[0];
    a[1] = ar[64];
    float2 s8n = make_float2(0.0f, 0.0f);
    float4 s8q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    constexpr int EV = EK == PF_Q4K ? 7 : 5;
#pragma unroll
    for (int kc = 0; kc < 8; kc++) {
        const float2 s8 = s8n;
        const float4 s8l = s8q;
        // outputs of step kc: 2 (kc - 1), +1 for kc = 1..6 (d8 pair kc - 1), 12..15 for kc = 7
        if (kc < 6) s8n = *reinterpret_cast<const float2 *>(pd8 + 8 * (kc >> 1) + 2 * (kc & 1));
        else if (kc == 6) s8q = *reinterpret_cast<const float4 *>(pd8 + 24);
        if (kc + 2 < 8) a[(kc + 2) % 3] = ar[64 * (kc + 2)];
        const int nreads = 1 + (kc + 2 < 8);
        if (nreads == 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[kc % 3], b0[kc], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[kc % 3], b1[kc], c1, 0, 0, 0);
        if (kc >= 1 && kc <= 6) {
            const float s8v[2] = {s8.x, s8.y};
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int v = 2 * (kc - 1) + r;
                pacc[v] = pf_epilogue<EK>(pacc[v], p0[v], p1[v], pcm[v], pdd, pdm, s8v[r]);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, EV, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, EV, 0);
        } else if (kc == 7) {
            const float s8v[4] = {s8l.x, s8l.y, s8l.z, s8l.w};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int v = 12 + r;
                pacc[v] = pf_epilogue<EK>(pacc[v], p0[v], p1[v], pcm[v], pdd, pdm, s8v[r]);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2 * EV, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2 * EV, 0);
        } else {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
    }
}

// Zero the first `bytes` of the workgroup's LDS (16-byte stores; bytes a multiple of 16), then a barrier.
__device__ __forceinline__ void pf_probe_fill(uint8_t *lds, int bytes, int tid) {
    for (int o = 16 * tid; o < bytes; o += 16 * PF_THREADS) *reinterpret_cast<uint4 *>(lds + o) = make_uint4(0, 0, 0, 0);
    __syncthreads();
}

// PROBE: the same kernel without its staging (no copies, no per-block wait and barrier; LDS zero-filled once) and
// with c null (nothing stored), which times the inner loop alone on the real grid (trhip_prefill_probe).
template <bool ACC, bool FAST, bool PROBE = false>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_q4k(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const int8_t *__restrict__ qt, const float *__restrict__ dt, const uint16_t *__restrict__ st,
    const uint8_t *__restrict__ bad_blk, float *__restrict__ c) {
    using T = Pf;
    constexpr int TM = T::TM, STAGE = T::STAGE, MT = PF_MT, EK = FAST ? PF_Q4K_FAST : PF_Q4K;
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowstate = reinterpret_cast<int *>(lds + T::DOFF + 3 * T::D);  // [TM] 0 ok, 1 NaN/Inf row, 2 outside M
    int *anybad = rowstate + TM;

    const int nb = (int)p.nb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + TM - 1) / TM, (N + PF_TN - 1) / PF_TN, tmi, tni);
    const int64_t n0 = tni * PF_TN, m0 = tmi * TM, mt0 = m0 >> 5;
    tile_row_flags<TM, PF_THREADS>(bad_blk, m0, M, nb, rowstate, anybad);

    // this wave's weight rows: lane l holds row 32 w + l % 32, code bytes 64 (l / 32) + 16 g .. +15 of each block
    // (elements 16 (l / 32) .. +15 of sub-blocks 2 g (low nibbles) and 2 g + 1 (high nibbles))
    const int nloc = 32 * w + (lane & 31);
    // buffers (the launcher checks that every offset fits 32 bits): the tiled activations over rows padded to a
    // multiple of TM, and the store's rows up to row0 + N
    const int64_t mpad = (M + TM - 1) / TM * TM;
    const dma_rsrc rq = dma_desc(qt, (uint32_t)(mpad * nb * 256));
    const dma_rsrc rs = dma_desc(st, (uint32_t)(mpad * nb * 32));
    const dma_rsrc rd = dma_desc(dt, (uint32_t)(mpad * nb * 4));
    const dma_rsrc rwq = dma_desc(p.qs, (uint32_t)((row0 + N) * nb * 128));
    const dma_rsrc rwh = dma_desc(p.aux, (uint32_t)((row0 + N) * nb * 16));
    // weight DMA: codes of 8 rows per instruction, lane j moving a 16-byte piece of row j / 8 to LDS slot j % 8, so
    // each instruction reads eight whole 128-byte row segments. Slot s of row r holds piece s ^ ((r / 2) % 8): the
    // 16 rows a b128 operand read pass covers then hit 16 different bank groups (rows are 128 bytes, so rows r and
    // r + 8 would share banks under a swizzle by r % 8). Headers by dwords, 16 rows per instruction.
    // (rows past row0 + N read zeros from the buffer's bound; their outputs are not stored)
    const int64_t wr0 = row0 + n0 + 32 * w;  // this wave's first weight row
    const uint32_t wq0 = (uint32_t)(wr0 * nb * 128), wh0 = (uint32_t)(wr0 * nb * 16);  // wave-uniform

    // stage block b into buffer buf: 1 KB activation pieces i (i < 8 MT codes of tile i / 8, chunk i % 8, then MT
    // msum pieces) dealt round-robin to the waves, the d8 pieces (256 bytes, two tiles each) after them, and each
    // wave's own weight rows. The per-lane offsets are rebuilt from a lane id the compiler cannot hoist, so no
    // register holds them across the block's tiles.
    auto stage = [&](int b, int buf) {
        const uint32_t ln = opaque((uint32_t)lane);
        const uint32_t v16 = 16 * ln;                                       // activation pieces
        const uint32_t vd = (ln >> 5) * (uint32_t)nb * 128 + 4 * (ln & 31);  // d8 pieces
        const uint32_t jr = ln >> 3, jc = ln & 7;
        // row 8 q + jr of the wave: piece jc ^ (jr / 2) ^ 4 (q % 2)
        const uint32_t vq0 = jr * (uint32_t)nb * 128 + 16 * (jc ^ (jr >> 1)), vq1 = vq0 ^ 64;
        const uint32_t vh = (ln >> 2) * (uint32_t)nb * 16 + 4 * (ln & 3);
        uint8_t *sb = lds + buf * STAGE;
        uint8_t *db = lds + T::DOFF + (b % 3) * T::D;
        // piece i = w + 8 j of the round-robin deal: chunk w of tile j (j < MT), then msum piece w (w < MT), and the
        // d8 pieces, pieces 9 MT + i, to waves (9 MT + i) % 8 (wave-uniform scalar arithmetic, no branch per piece)
        static_assert(PF_W == 8 && MT <= PF_W && T::PIECES == 9 * MT, "one chunk per wave and tile");
#pragma unroll
        for (int t = 0; t < MT; t++)
            dma16(rq, lds_addr(sb + 1024 * (8 * t + w)), v16, (uint32_t)((((mt0 + t) * nb + b) * 8 + w) * 1024));
        if (w < MT) dma16(rs, lds_addr(sb + T::A + 1024 * w), v16, (uint32_t)(((mt0 + w) * nb + b) * 1024));
#pragma unroll
        for (int i = 0; i < MT / 2; i++)
            if ((T::PIECES + i) % PF_W == w)
                dma4(rd, lds_addr(db + 256 * i), vd, (uint32_t)(((mt0 + 2 * i) * nb + b) * 128));
        uint8_t *wb = sb + T::A + T::S + w * T::WREG;
#pragma unroll
        for (int q = 0; q < 2; q++) dma4(rwh, lds_addr(wb + 256 * q), vh, wh0 + (uint32_t)(16 * b + 256 * q * nb));
#pragma unroll
        for (int q = 0; q < 4; q++)
            dma16(rwq, lds_addr(wb + 512 + 1024 * q), (q & 1) ? vq1 : vq0, wq0 + (uint32_t)(128 * b + 1024 * q * nb));
    };

    if (PROBE)
        pf_probe_fill(lds, T::DOFF + 3 * T::D, tid);
    else
        stage(0, 0);

    float accf[MT][16];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) accf[t][v] = 0.0f;
    // Pending epilogue state (the tile before the one whose MFMAs run): sums (in set y, or x), msum, d, dmin. Before
    // the first block nothing is pending: zero sums and msum with zero d8 (slot 2, zeroed here) add +-0 to accf =
    // +0, which stays +0.
    v16i x0 = (v16i){0}, x1 = (v16i){0}, y0 = (v16i){0}, y1 = (v16i){0};
    v16f pca = (v16f){0.0f}, pcb = (v16f){0.0f};  // msum of tiles 0, 2 (pca) and 1, 3 (pcb)
    float pdd = 0.0f, pdm = 0.0f;
    if (tid < T::D / 4) reinterpret_cast<float *>(lds + T::DOFF + 2 * T::D)[tid] = 0.0f;
    const int lrow = 4 * (lane >> 5);  // this lane's d8 offset within a tile

    for (int b = 0; b < nb; b++) {
        // this wave's loads of block b have landed; after the barrier everyone's have, and nobody reads the other
        // buffer (block b - 1) any more
        if (!PROBE) {
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (b + 1 < nb) stage(b + 1, (b + 1) & 1);
        }
        const uint8_t *sb = lds + (b & 1) * STAGE;

        // weight block b from LDS: scales and both planes of all eight sub-blocks
        const uint8_t *wb = sb + T::A + T::S + w * T::WREG;
        // (addresses recomputed per block from a lane id the compiler cannot hoist: no registers held across blocks)
        const int ln = (int)opaque((uint32_t)lane), r = ln & 31, h = ln >> 5;
        const uint4 wh = *reinterpret_cast<const uint4 *>(wb + 16 * r);
        uint4 wq[4];  // pieces 4 h + g of row r
        const uint8_t *wrb = wb + 512 + 128 * r;
#pragma unroll
        for (int g = 0; g < 4; g++) wq[g] = *reinterpret_cast<const uint4 *>(wrb + 16 * ((4 * h + g) ^ ((r >> 1) & 7)));
        uint32_t sc_lo, sc_hi, m_lo, m_hi;
        q4k_scales(wh.y, wh.z, wh.w, sc_lo, sc_hi, m_lo, m_hi);
        const float dd = f16_to_f32((uint16_t)(wh.x & 0xFFFF)), dm = f16_to_f32((uint16_t)(wh.x >> 16));
        v4i b0[8], b1[8];
#pragma unroll
        for (int kc = 0; kc < 8; kc++) {
            const uint4 raw = wq[kc >> 1];
            const uint4 nib = (kc & 1) ? make_uint4((raw.x >> 4) & 0x0F0F0F0Fu, (raw.y >> 4) & 0x0F0F0F0Fu,
                                                    (raw.z >> 4) & 0x0F0F0F0Fu, (raw.w >> 4) & 0x0F0F0F0Fu)
                                       : make_uint4(raw.x & 0x0F0F0F0Fu, raw.y & 0x0F0F0F0Fu, raw.z & 0x0F0F0F0Fu,
                                                    raw.w & 0x0F0F0F0Fu);
            const uint32_t sc = ((kc < 4 ? sc_lo : sc_hi) >> (8 * (kc & 3))) & 0xFF;
            b0[kc] = mul16(nib, sc & 7);
            b1[kc] = mul16(nib, sc >> 3);
        }
        // msum B operand of this lane's row: [64 m_0..7 | m_0..7] (lanes < 32 hold k 0..7, lanes >= 32 k 8..15)
        const v8h bmv = small_f16x8(m_lo, m_hi, (lane >> 5) ? (_Float16)1.0f : (_Float16)64.0f);

        // (every LDS address below derives from ln, so none is hoisted out of the loop and held in a register)
        const v4i *ar = reinterpret_cast<const v4i *>(sb) + ln;  // tile t, chunk kc: + 512 t + 64 kc
        const v8h *am = reinterpret_cast<const v8h *>(sb + T::A) + ln;  // tile t: + 64 t
        const float *d8b = reinterpret_cast<const float *>(lds + T::DOFF + (b % 3) * T::D) + 4 * h;
        const float *d8p = reinterpret_cast<const float *>(lds + T::DOFF + ((b + 2) % 3) * T::D) + 4 * h;
        // tiles 0..3 in sets x, y, x, y; each one's epilogue runs inside the next tile. A tile's msum MFMA is issued
        // before its int8 MFMAs, into the msum set the pending epilogue does not read, so it has completed long
        // before that tile's own epilogue reads it
        pca = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[0], bmv, (v16f){0.0f}, 0, 0, 0);
        pf_tile<EK>(x0, x1, y0, y1, pcb, pdd, pdm, accf[MT - 1], d8p + 32 * (MT - 1), ar, b0, b1);
        pdd = dd;
        pdm = dm;
        pcb = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[64], bmv, (v16f){0.0f}, 0, 0, 0);
        pf_tile<EK>(y0, y1, x0, x1, pca, pdd, pdm, accf[0], d8b, ar + 512, b0, b1);
        pca = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[128], bmv, (v16f){0.0f}, 0, 0, 0);
        pf_tile<EK>(x0, x1, y0, y1, pcb, pdd, pdm, accf[1], d8b + 32, ar + 1024, b0, b1);
        pcb = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[192], bmv, (v16f){0.0f}, 0, 0, 0);
        pf_tile<EK>(y0, y1, x0, x1, pca, pdd, pdm, accf[2], d8b + 64, ar + 1536, b0, b1);
    }
    {  // the last block's last tile (set y, msum pcb)
        const float *d8l = reinterpret_cast<const float *>(lds + T::DOFF + ((nb + 2) % 3) * T::D) + lrow + 32 * (MT - 1);
#pragma unroll
        for (int v = 0; v < 16; v++)
            accf[MT - 1][v] = pf_epilogue<EK>(accf[MT - 1][v], y0[v], y1[v], pcb[v], pdd, pdm, d8l[8 * (v >> 2) + (v & 3)]);
    }

    const int64_t gn = n0 + nloc;
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int mloc = 32 * t + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            if ((!PROBE || c) && gn < N && rowstate[mloc] == 0) {
                float *o = c + (m0 + mloc) * N + gn;
                *o = ACC ? *o + accf[t][v] : accf[t][v];
            }
        }
    }
    // rows holding NaN/Inf take the exact fp32 path (quantGemv) on their own; rare
    if (!*anybad) return;
    for (int i = tid; i < TM * PF_TN; i += PF_THREADS) {
        const int ml = i / PF_TN, nl = i % PF_TN;
        const int64_t gn2 = n0 + nl;
        if (rowstate[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = exact_dot_row<kQ4K>(p, row0 + gn2, x + gm * K, K);
        float *o = c + gm * N + gn2;
        *o = ACC ? *o + v : v;
    }
}


// q6_k (tensor/cpu_quant_q8.go:378-407). Per block, the wave's 32 weight rows' signed products
// v = (q6 - 32) sc_j (the sub-block scale folded in; |v| <= 4096) are split as v = 128 h + l, h = v >> 7 in
// [-32, 32] and l = v & 127 in [0, 127], both int8, so X = isum - 32 msum = sum v q8 = 128 sum h q8 + sum l q8:
// two int8 MFMA accumulations over the whole block (l into the first set, h into the second) and the reference's
// epilogue t = fl(d fl(X)), acc = fl(acc + fl(t d8)). Tiles, accumulator sets and the delayed epilogue are those of
// prefill_q4k; there is no minimum term. The activation buffers are double-buffered as there; each wave's weight
// rows have one buffer, refilled with the next block as soon as the wave has read the current one into registers.
struct Pf6 {
    static constexpr int TM = 32 * PF_MT;
    static constexpr int A = PF_MT * 8192;                  // activation codes of one block (two buffers)
    static constexpr int SC = 0, QL = 512, QH = QL + 4096;   // one wave's rows: 32 x 16 scales, 32 x 128 ql, 32 x 64 qh
    static constexpr int WREG = QH + 2048;
    static constexpr int W = 2 * A;                          // the waves' weight buffers
    static constexpr int D = PF_MT * 128;                    // d8 of one block (slot b % 3, read one block later)
    static constexpr int DOFF = W + PF_W * WREG;
    static constexpr size_t LDS = DOFF + 3 * D + (TM + 1) * sizeof(int);
};
static_assert(Pf6::LDS <= 160 * 1024, "one workgroup per CU");

typedef short pf_s2 __attribute__((ext_vector_type(2)));

// Chunk kc's two B operands for lane (r, h): elements 32 kc + 16 h .. + 15 of the row, the four 4-element groups
// e = 2 tt + hh (tt, hh in 0..1) from ql dword L[e] (nibble half k / 2) and qh dword H[e] (bit pair k = kc % 4), all
// in sub-block 2 kc + h with signed scale sc. Per group: the codes c as bytes, spread to 16-bit pairs, v = c sc - 32 sc
// by packed 16-bit multiply-adds, then the bytes of v >> 7 (h) and of v & 127 (l).
__device__ __forceinline__ void q6_planes(const uint32_t (&L)[4], const uint32_t (&H)[4], int k, int sc, v4i &lo,
                                          v4i &hi) {
    const pf_s2 S = (pf_s2){(short)sc, (short)sc}, O = (pf_s2){(short)(-32 * sc), (short)(-32 * sc)};
    uint32_t lb[4], hb[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t lw = (k >> 1) ? (L[e] >> 4) : L[e];
        const uint32_t hw = k == 0 ? (H[e] << 4) : k == 1 ? (H[e] << 2) : k == 2 ? H[e] : (H[e] >> 2);
        const uint32_t C = (lw & 0x0F0F0F0Fu) | (hw & 0x30303030u);  // codes 0..63
        const pf_s2 c01 = __builtin_bit_cast(pf_s2, __builtin_amdgcn_perm(0u, C, 0x0c010c00u));
        const pf_s2 c23 = __builtin_bit_cast(pf_s2, __builtin_amdgcn_perm(0u, C, 0x0c030c02u));
        const uint32_t v01 = __builtin_bit_cast(uint32_t, c01 * S + O), v23 = __builtin_bit_cast(uint32_t, c23 * S + O);
        lb[e] = __builtin_amdgcn_perm(v23, v01, 0x06040200u) & 0x7F7F7F7Fu;  // low bytes, low 7 bits: v & 127
        hb[e] = __builtin_amdgcn_perm(v23 >> 7, v01 >> 7, 0x06040200u);     // bits 7..14 of each v: v >> 7
    }
    lo = (v4i){(int)lb[0], (int)lb[1], (int)lb[2], (int)lb[3]};
    hi = (v4i){(int)hb[0], (int)hb[1], (int)hb[2], (int)hb[3]};
}

template <bool ACC, bool PROBE = false>  // PROBE: as for prefill_q4k
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_q6k(
    const Planes p, int64_t N, int64_t row0, int64_t M, int64_t K, const float *__restrict__ x,
    const int8_t *__restrict__ qt, const float *__restrict__ dt, const uint8_t *__restrict__ bad_blk,
    float *__restrict__ c) {
    using T = Pf6;
    constexpr int TM = T::TM, MT = PF_MT;
    extern __shared__ __align__(16) uint8_t lds[];
    int *rowstate = reinterpret_cast<int *>(lds + T::DOFF + 3 * T::D);  // [TM] 0 ok, 1 NaN/Inf row, 2 outside M
    int *anybad = rowstate + TM;

    const int nb = (int)p.nb;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int64_t tmi, tni;
    tile_of(blockIdx.x, (M + TM - 1) / TM, (N + PF_TN - 1) / PF_TN, tmi, tni);
    const int64_t n0 = tni * PF_TN, m0 = tmi * TM, mt0 = m0 >> 5;
    tile_row_flags<TM, PF_THREADS>(bad_blk, m0, M, nb, rowstate, anybad);

    const int nloc = 32 * w + (lane & 31);  // this lane's weight row (as the B operand: column lane % 32)
    const int64_t mpad = (M + TM - 1) / TM * TM;
    const dma_rsrc rq = dma_desc(qt, (uint32_t)(mpad * nb * 256));
    const dma_rsrc rd = dma_desc(dt, (uint32_t)(mpad * nb * 4));
    const dma_rsrc rwl = dma_desc(p.qs, (uint32_t)((row0 + N) * nb * 128));
    const dma_rsrc rwh = dma_desc(p.aux, (uint32_t)((row0 + N) * nb * 64));
    const dma_rsrc rws = dma_desc(p.sc, (uint32_t)((row0 + N) * nb * 16));
    // this wave's rows (rows past row0 + N read zeros from the buffers' bounds; their outputs are not stored)
    const int64_t wr0 = row0 + n0 + 32 * w;
    const uint32_t wl0 = (uint32_t)(wr0 * nb * 128), wh0 = (uint32_t)(wr0 * nb * 64), ws0 = (uint32_t)(wr0 * nb * 16);
    uint8_t *wb = lds + T::W + w * T::WREG;
    // d of this lane's row, one block ahead in a register (plain loads)
    const int64_t drow = wr0 + (lane & 31) < row0 + N ? wr0 + (lane & 31) : row0 + N - 1;
    const uint16_t *dp = p.d + drow * nb;

    // activation codes (tile t chunk w per wave) and the d8 pieces (two tiles each, waves 0 .. MT / 2 - 1) of block
    // b into buffer buf, as in prefill_q4k
    auto stage_act = [&](int b, int buf) {
        const uint32_t ln = opaque((uint32_t)lane);
        const uint32_t v16 = 16 * ln, vd = (ln >> 5) * (uint32_t)nb * 128 + 4 * (ln & 31);
        uint8_t *sb = lds + buf * T::A;
        uint8_t *db = lds + T::DOFF + (b % 3) * T::D;
#pragma unroll
        for (int t = 0; t < MT; t++)
            dma16(rq, lds_addr(sb + 1024 * (8 * t + w)), v16, (uint32_t)((((mt0 + t) * nb + b) * 8 + w) * 1024));
        if (w < MT / 2) dma4(rd, lds_addr(db + 256 * w), vd, (uint32_t)(((mt0 + 2 * w) * nb + b) * 128));
    };
    // this wave's rows of block b: scales by dwords (16 rows per instruction); ql as prefill_q4k's codes (eight rows
    // per instruction, slot s of row r holding piece s ^ ((r / 2) % 8)); qh 16 rows per instruction, slot s of row r
    // holding piece s ^ ((r / 4) % 4), so that the 16 rows a b128 read pass covers hit 16 different bank groups
    auto stage_w = [&](int b) {
        const uint32_t ln = opaque((uint32_t)lane);
        const uint32_t vs = (ln >> 2) * (uint32_t)nb * 16 + 4 * (ln & 3);
        const uint32_t jr = ln >> 3, jc = ln & 7;
        const uint32_t vl0 = jr * (uint32_t)nb * 128 + 16 * (jc ^ (jr >> 1)), vl1 = vl0 ^ 64;
        const uint32_t hr = ln >> 2, hc = ln & 3;
        const uint32_t vh = hr * (uint32_t)nb * 64 + 16 * (hc ^ ((hr >> 2) & 3));
#pragma unroll
        for (int q = 0; q < 2; q++) dma4(rws, lds_addr(wb + T::SC + 256 * q), vs, ws0 + (uint32_t)(16 * b + 256 * q * nb));
#pragma unroll
        for (int q = 0; q < 4; q++)
            dma16(rwl, lds_addr(wb + T::QL + 1024 * q), (q & 1) ? vl1 : vl0, wl0 + (uint32_t)(128 * b + 1024 * q * nb));
#pragma unroll
        for (int q = 0; q < 2; q++)
            dma16(rwh, lds_addr(wb + T::QH + 1024 * q), vh, wh0 + (uint32_t)(64 * b + 1024 * q * nb));
    };

    uint16_t draw = 0x3C00;  // (the probe's d: 1.0)
    if (PROBE) {
        pf_probe_fill(lds, T::DOFF + 3 * T::D, tid);
    } else {
        stage_act(0, 0);
        stage_w(0);
        draw = dp[0];
    }

    float accf[MT][16];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) accf[t][v] = 0.0f;
    // pending epilogue state as in prefill_q4k (nothing pending before the first block: zero sums, zero d8)
    v16i x0 = (v16i){0}, x1 = (v16i){0}, y0 = (v16i){0}, y1 = (v16i){0};
    const v16f nocm = (v16f){0.0f};
    float pdd = 0.0f;
    if (tid < T::D / 4) reinterpret_cast<float *>(lds + T::DOFF + 2 * T::D)[tid] = 0.0f;
    const int lrow = 4 * (lane >> 5);

    for (int b = 0; b < nb; b++) {
        if (!PROBE) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // d of block b (loaded during the previous block) is used before the next copies are issued, so the wait the
        // compiler places for that load cannot fall after them
        const float dd = f16_to_f32(draw);
        asm volatile("" ::"v"(dd));
        if (!PROBE && b + 1 < nb) stage_act(b + 1, (b + 1) & 1);
        const uint8_t *sb = lds + (b & 1) * T::A;

        // this lane's bytes of the block: ql pieces 4 h + g, qh pieces 2 h + tt, the row's 16 scales
        const int ln = (int)opaque((uint32_t)lane), r = ln & 31, h = ln >> 5;
        uint4 wq[4], qq[2];
#pragma unroll
        for (int g = 0; g < 4; g++)
            wq[g] = *reinterpret_cast<const uint4 *>(wb + T::QL + 128 * r + 16 * ((4 * h + g) ^ ((r >> 1) & 7)));
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
            qq[tt] = *reinterpret_cast<const uint4 *>(wb + T::QH + 64 * r + 16 * ((2 * h + tt) ^ ((r >> 2) & 3)));
        const uint4 scw = *reinterpret_cast<const uint4 *>(wb + T::SC + 16 * r);
        // every read of the buffer has landed: refill it with the next block, and load its d
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (!PROBE) {
            if (b + 1 < nb) stage_w(b + 1);
            draw = dp[b + 1 < nb ? b + 1 : b];
        }
        v4i b0[8], b1[8];
#pragma unroll
        for (int kc = 0; kc < 8; kc++) {
            const int n2 = kc >> 2, k = kc & 3, kk = k & 1;
            uint32_t L[4], H[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint4 lq = wq[n2 + 2 * (e >> 1)], hq = qq[e >> 1];
                const int ld = 2 * kk + (e & 1), hd = 2 * n2 + (e & 1);
                L[e] = ld == 0 ? lq.x : ld == 1 ? lq.y : ld == 2 ? lq.z : lq.w;
                H[e] = hd == 0 ? hq.x : hd == 1 ? hq.y : hd == 2 ? hq.z : hq.w;
            }
            const uint32_t sw = (kc >> 1) == 0 ? scw.x : (kc >> 1) == 1 ? scw.y : (kc >> 1) == 2 ? scw.z : scw.w;
            const int sc = __builtin_amdgcn_sbfe((int)sw, 16 * (kc & 1) + 8 * h, 8);  // sub-block 2 kc + h
            q6_planes(L, H, k, sc, b0[kc], b1[kc]);
        }

        const v4i *ar = reinterpret_cast<const v4i *>(sb) + ln;  // tile t, chunk kc: + 512 t + 64 kc
        const float *d8b = reinterpret_cast<const float *>(lds + T::DOFF + (b % 3) * T::D) + 4 * h;
        const float *d8p = reinterpret_cast<const float *>(lds + T::DOFF + ((b + 2) % 3) * T::D) + 4 * h;
        pf_tile<PF_Q6K>(x0, x1, y0, y1, nocm, pdd, 0.0f, accf[MT - 1], d8p + 32 * (MT - 1), ar, b0, b1);
        pdd = dd;
        pf_tile<PF_Q6K>(y0, y1, x0, x1, nocm, pdd, 0.0f, accf[0], d8b, ar + 512, b0, b1);
        pf_tile<PF_Q6K>(x0, x1, y0, y1, nocm, pdd, 0.0f, accf[1], d8b + 32, ar + 1024, b0, b1);
        pf_tile<PF_Q6K>(y0, y1, x0, x1, nocm, pdd, 0.0f, accf[2], d8b + 64, ar + 1536, b0, b1);
    }
    {  // the last block's last tile (set y)
        const float *d8l = reinterpret_cast<const float *>(lds + T::DOFF + ((nb + 2) % 3) * T::D) + lrow + 32 * (MT - 1);
#pragma unroll
        for (int v = 0; v < 16; v++)
            accf[MT - 1][v] = pf_epilogue<PF_Q6K>(accf[MT - 1][v], y0[v], y1[v], 0.0f, pdd, 0.0f, d8l[8 * (v >> 2) + (v & 3)]);
    }

    const int64_t gn = n0 + nloc;
#pragma unroll
    for (int t = 0; t < MT; t++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int mloc = 32 * t + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            if ((!PROBE || c) && gn < N && rowstate[mloc] == 0) {
                float *o = c + (m0 + mloc) * N + gn;
                *o = ACC ? *o + accf[t][v] : accf[t][v];
            }
        }
    }
    // rows holding NaN/Inf take the exact fp32 path (quantGemv) on their own; rare
    if (!*anybad) return;
    for (int i = tid; i < TM * PF_TN; i += PF_THREADS) {
        const int ml = i / PF_TN, nl = i % PF_TN;
        const int64_t gn2 = n0 + nl;
        if (rowstate[ml] != 1 || gn2 >= N) continue;
        const int64_t gm = m0 + ml;
        const float v = exact_dot_row<kQ6K>(p, row0 + gn2, x + gm * K, K);
        float *o = c + gm * N + gn2;
        *o = ACC ? *o + v : v;
    }
}
}  // namespace

// Taken when the grid of 128 x 256 tiles has at least 192 workgroups (one per CU fits), else the 64-row kernel of
// actq_mfma.hip keeps more of the device busy.
namespace {
// every buffer offset of the kernel fits 32 bits (tiled activations, the store's rows up to row0 + N)
bool prefill_fits32(int64_t M, int64_t N, int64_t row0, int64_t K) {
    const int64_t mpad = (M + Pf::TM - 1) / Pf::TM * Pf::TM, nb = K / 256;
    return mpad * nb * 256 < ((int64_t)1 << 32) && (row0 + N + PF_TN) * nb * 128 < ((int64_t)1 << 32);
}
}  // namespace

bool prefill_tiles_apply(int dtype, int64_t M, int64_t N, int64_t row0, int64_t K) {
    if ((dtype != kQ4K && dtype != kQ6K) || !prefill_fits32(M, N, row0, K)) return false;
    const int64_t wgs = ((M + Pf::TM - 1) / Pf::TM) * ((N + PF_TN - 1) / PF_TN);
    return M >= 256 && wgs >= 192;
}

int launch_prefill_q4k(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                       int64_t M, bool acc, const int8_t *qt, const float *dt, const uint16_t *st, const uint8_t *bad,
                       bool fast) {
    using T = Pf;
    static_assert(T::TM == kPrefillRowPad, "the tiled layout pads rows to one workgroup row tile");
    const int64_t wgs = ((M + T::TM - 1) / T::TM) * ((N + PF_TN - 1) / PF_TN);
    if (wgs >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "prefill: grid too large");
    if (!prefill_fits32(M, N, row0, w->K)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "prefill: buffers above 4 GB");
    auto go = [&](auto kern) {
        int st0 = allow_dyn_lds(ctx, reinterpret_cast<const void *>(kern), T::LDS, "prefill: LDS size");
        if (st0 != TRHIP_OK) return st0;
        hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(PF_THREADS), T::LDS, ctx->stream, w->planes(), N, row0, M,
                           w->K, x, qt, dt, st, bad, c);
        return launch_check(ctx, "prefill_q4k");
    };
    if (fast) return acc ? go(&prefill_q4k<true, true>) : go(&prefill_q4k<false, true>);
    return acc ? go(&prefill_q4k<true, false>) : go(&prefill_q4k<false, false>);
}

int launch_prefill_q6k(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                       int64_t M, bool acc, const int8_t *qt, const float *dt, const uint8_t *bad) {
    using T = Pf6;
    static_assert(T::TM == kPrefillRowPad, "the tiled layout pads rows to one workgroup row tile");
    const int64_t wgs = ((M + T::TM - 1) / T::TM) * ((N + PF_TN - 1) / PF_TN);
    if (wgs >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "prefill: grid too large");
    if (!prefill_fits32(M, N, row0, w->K)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "prefill: buffers above 4 GB");
    auto go = [&](auto kern) {
        int st0 = allow_dyn_lds(ctx, reinterpret_cast<const void *>(kern), T::LDS, "prefill: LDS size");
        if (st0 != TRHIP_OK) return st0;
        hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(PF_THREADS), T::LDS, ctx->stream, w->planes(), N, row0, M,
                           w->K, x, qt, dt, bad, c);
        return launch_check(ctx, "prefill_q6k");
    };
    return acc ? go(&prefill_q6k<true>) : go(&prefill_q6k<false>);
}

int launch_prefill_probe(trhip_ctx *ctx, int kind, int64_t M, int64_t N, int64_t K) {
    if (kind < 0 || kind > 2 || M <= 0 || N <= 0 || K <= 0 || K % 256 != 0)
        return fail(ctx, TRHIP_ERR_INVALID, "prefill_probe: kind 0..2, M, N > 0 and K a positive multiple of 256");
    if (capturing(ctx)) return fail(ctx, TRHIP_ERR_INVALID, "prefill_probe: not capturable");
    const int64_t nb = K / 256, TM = Pf::TM;
    const int64_t wgs = ((M + TM - 1) / TM) * ((N + PF_TN - 1) / PF_TN);
    if (wgs >= ((int64_t)1 << 31)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "prefill_probe: grid too large");
    // the row flags the kernels read (every activation row finite); weights and activations are not read
    int st = TRHIP_OK;
    uint8_t *flags = static_cast<uint8_t *>(workspace(ctx, (size_t)(M * nb), &st));
    if (!flags) return st;
    hipError_t e = hipMemsetAsync(flags, 0, (size_t)(M * nb), ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "prefill_probe: flags");
    Planes pl{};
    pl.nb = nb;
    auto go = [&](auto kern, size_t lds) {
        int st0 = allow_dyn_lds(ctx, reinterpret_cast<const void *>(kern), lds, "prefill_probe: LDS size");
        if (st0 != TRHIP_OK) return st0;
        return 0;
    };
    if (kind == 2) {
        if ((st = go(&prefill_q6k<false, true>, Pf6::LDS)) != TRHIP_OK) return st;
        hipLaunchKernelGGL((prefill_q6k<false, true>), dim3((unsigned)wgs), dim3(PF_THREADS), Pf6::LDS, ctx->stream, pl,
                           N, (int64_t)0, M, K, nullptr, nullptr, nullptr, flags, nullptr);
    } else if (kind == 1) {
        if ((st = go(&prefill_q4k<false, true, true>, Pf::LDS)) != TRHIP_OK) return st;
        hipLaunchKernelGGL((prefill_q4k<false, true, true>), dim3((unsigned)wgs), dim3(PF_THREADS), Pf::LDS, ctx->stream,
                           pl, N, (int64_t)0, M, K, nullptr, nullptr, nullptr, nullptr, flags, nullptr);
    } else {
        if ((st = go(&prefill_q4k<false, false, true>, Pf::LDS)) != TRHIP_OK) return st;
        hipLaunchKernelGGL((prefill_q4k<false, false, true>), dim3((unsigned)wgs), dim3(PF_THREADS), Pf::LDS, ctx->stream,
                           pl, N, (int64_t)0, M, K, nullptr, nullptr, nullptr, nullptr, flags, nullptr);
    }
    return launch_check(ctx, "prefill_probe");
}

}  // namespace trhip
