// gemm_rows.hip -- fp32-activation quant matmul for M > 1, bit-identical to TR's CPU order.
//
// tensor/cpu_quant.go:103-147 (quantGemmPanels) and the tile path (:59-82, gemmPart in
// cpu_matmul.go:330-380) both compute, for every output (m, n): for each 256-deep K chunk a fresh
// fused chain from +0 in ascending k (sgemm6x16, cpu_micro_amd64.s:14-64), the chunk results added
// in chunk order into a cleared `part`, then c[m, n] += part.
//
// Mapping: a wave is 64 weight rows (lane = row) on one 256-deep chunk. It decodes its rows' weights 32 elements at
// a time, exactly as tensor/quant.go does, and advances the chains of up to 16 activation rows with K = 1 matrix
// instructions, each of whose outputs is one fused multiply-add. A wave's 64 row images of a chunk are loaded with
// whole cache lines per instruction and staged in LDS, where each lane reads its own row back; the activations of a
// group are staged the same way. A workgroup is kStageWaves (or, for grids of few row blocks, 4) such waves on
// consecutive chunks of the same 64 rows. Their chain results are added to `part` in chunk order in LDS, or, when
// the chunks of a row block are split over several workgroups, written out per chunk and added in chunk order by
// a second kernel.
#include "trhip_internal.hpp"

#include <type_traits>

namespace trhip {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
// Plain vector types for registers carried across loop iterations (the HIP uint4 / float4 structs are copied with
// memcpy, which keeps them in private memory there).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kStageWaves = 8;  // chunk-waves per workgroup when one workgroup covers a row block's chunks
constexpr int kSplitWaves = 4;  // chunk-waves per workgroup when a row block's chunks are split over workgroups
constexpr int kXPitch = 36;     // floats per activation row of a staged 32-wide group: rows land on distinct banks
constexpr int kRPitch = 68;     // floats per row of a wave's 16 x 64 chain results

// f(integral_constant<int, I>) for I = B .. E - 1, so that loop indices are constants in the body.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// 32 consecutive elements (group G of a 32-element grid along the row) of one block, decoded exactly as
// tensor/quant.go:139-205.
template <int DT>
struct Group;

template <>
struct Group<kQ8> {
    uint4 a, b;
    uint32_t d;
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

// A weight row's bytes for one 256-wide chunk, as the 16-byte pieces of an LDS image. A wave loads the 64 rows'
// images with consecutive lanes on consecutive pieces of a row (whole cache lines per instruction) and then reads
// its own row back, a lane per row. kPitch (bytes per row image) keeps 16 consecutive rows on distinct LDS banks.
template <int DT>
struct Image;

template <>
struct Image<kQ8> {  // 8 blocks x 32 codes, then the 8 fp16 scales
    static constexpr int kPieces = 16, kPitch = 272, kScaleOff = 256, kBlocks = 8;
    __device__ static const uint8_t *piece(const Planes &p, int64_t b0, int q) { return p.qs + b0 * 32 + 16 * q; }
    __device__ static int piece_block(int q) { return q >> 1; }
};

template <>
struct Image<kQ4> {  // 8 blocks x 16 code bytes, then the 8 fp16 scales
    static constexpr int kPieces = 8, kPitch = 144, kScaleOff = 128, kBlocks = 8;
    __device__ static const uint8_t *piece(const Planes &p, int64_t b0, int q) { return p.qs + b0 * 16 + 16 * q; }
    __device__ static int piece_block(int q) { return q; }
};

template <>
struct Image<kQ4K> {  // the lane-sliced qs block (128), then the header d, dmin, scales (16)
    static constexpr int kPieces = 9, kPitch = 144, kScaleOff = -1, kBlocks = 1;
    __device__ static const uint8_t *piece(const Planes &p, int64_t b0, int q) {
        return q < 8 ? p.qs + b0 * 128 + 16 * q : p.aux + b0 * 16;
    }
    __device__ static int piece_block(int) { return 0; }
};

template <>
struct Image<kQ6K> {  // ql (128), qh (64), the 16 int8 scales (16); d stays in a register
    static constexpr int kPieces = 13, kPitch = 208, kScaleOff = -1, kBlocks = 1;
    __device__ static const uint8_t *piece(const Planes &p, int64_t b0, int q) {
        return q < 8 ? p.qs + b0 * 128 + 16 * q : q < 12 ? p.aux + b0 * 64 + 16 * (q - 8) : p.sc + b0 * 16;
    }
    __device__ static int piece_block(int) { return 0; }
};

// One wave's staging registers for the images of 64 rows: piece P = 64 i + lane is piece P % kPieces of row
// P / kPieces. Blocks past the end of a row (a short last chunk of q8_0 / q4_0) are neither loaded nor read.
template <int DT>
struct Stage {
    using I = Image<DT>;
    static constexpr int kScales = I::kScaleOff >= 0 ? 8 : 0;
    u32x4 w[I::kPieces];
    uint32_t s[kScales > 0 ? kScales : 1];
    uint32_t d6;  // q6_k: the fp16 scale of the lane's own row
    __device__ __forceinline__ void load(const Planes &p, int64_t row0, int64_t rbase, int64_t N, int64_t chunk,
                                         int lane) {
        const int64_t nblk = p.nb - chunk * I::kBlocks;  // blocks of the row from this chunk on
#pragma unroll
        for (int i = 0; i < I::kPieces; i++) {
            const int P = 64 * i + lane, rr = P / I::kPieces, q = P % I::kPieces;
            const int64_t row = row0 + (rbase + rr < N ? rbase + rr : N - 1);
            if (I::kBlocks == 1 || I::piece_block(q) < nblk)  // a k-quant chunk is one whole block
                w[i] = *reinterpret_cast<const u32x4 *>(I::piece(p, row * p.nb + chunk * I::kBlocks, q));
        }
#pragma unroll
        for (int i = 0; i < kScales; i++) {
            const int S = 64 * i + lane, rr = S >> 3, blk = S & 7;
            const int64_t row = row0 + (rbase + rr < N ? rbase + rr : N - 1);
            if (blk < nblk) s[i] = p.d[row * p.nb + chunk * 8 + blk];
        }
        if (DT == kQ6K) {
            const int64_t row = row0 + (rbase + lane < N ? rbase + lane : N - 1);
            d6 = p.d[row * p.nb + chunk];
        }
    }
    __device__ __forceinline__ void store(uint8_t *ws, int lane) const {
#pragma unroll
        for (int i = 0; i < I::kPieces; i++) {
            const int P = 64 * i + lane, rr = P / I::kPieces, q = P % I::kPieces;
            *reinterpret_cast<u32x4 *>(ws + rr * I::kPitch + 16 * q) = w[i];
        }
#pragma unroll
        for (int i = 0; i < kScales; i++) {
            const int S = 64 * i + lane, rr = S >> 3, blk = S & 7;
            *reinterpret_cast<uint16_t *>(ws + rr * I::kPitch + I::kScaleOff + 2 * blk) = (uint16_t)s[i];
        }
    }
};

// Group G of a row's chunk from its LDS image (the same bytes Group<DT>::load fetches from the planes).
template <int DT>
__device__ __forceinline__ void group_from_image(Group<DT> &g, const uint8_t *img, int G, uint32_t d6);

template <>
__device__ __forceinline__ void group_from_image<kQ8>(Group<kQ8> &g, const uint8_t *img, int G, uint32_t) {
    g.a = *reinterpret_cast<const uint4 *>(img + 32 * G);
    g.b = *reinterpret_cast<const uint4 *>(img + 32 * G + 16);
    g.d = *reinterpret_cast<const uint16_t *>(img + 256 + 2 * G);
}

template <>
__device__ __forceinline__ void group_from_image<kQ4>(Group<kQ4> &g, const uint8_t *img, int G, uint32_t) {
    g.a = *reinterpret_cast<const uint4 *>(img + 16 * G);
    g.d = *reinterpret_cast<const uint16_t *>(img + 128 + 2 * G);
}

template <>
__device__ __forceinline__ void group_from_image<kQ4K>(Group<kQ4K> &g, const uint8_t *img, int j, uint32_t) {
    g.h = *reinterpret_cast<const uint4 *>(img + 128);
    g.a = *reinterpret_cast<const uint4 *>(img + 16 * (j >> 1));
    g.b = *reinterpret_cast<const uint4 *>(img + 64 + 16 * (j >> 1));
}

template <>
__device__ __forceinline__ void group_from_image<kQ6K>(Group<kQ6K> &g, const uint8_t *img, int G, uint32_t d6) {
    const int n = G >> 2, k4 = G & 3;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        g.ql[t] = *reinterpret_cast<const uint2 *>(img + 16 * n + 8 * (k4 & 1) + 32 * t);
        g.qh[t] = *reinterpret_cast<const uint2 *>(img + 128 + 8 * n + 16 * t);
    }
    g.sc = *reinterpret_cast<const uint16_t *>(img + 192 + 8 * n + 2 * k4);
    g.d = d6;
}

// The chains of one pass of activation rows for a wave's 64 weight rows, advanced by a 32-wide group: lane l
// holds weight row l's decoded elements y[e] (the B operand) and reads the activations (the A operand) from the
// wave's 16 x 32 LDS tile. Both instructions are K = 1 outer products, each output one fma(a, b, c) with a single
// rounding (checked bit for bit against fmaf, subnormal, signed-zero and non-finite operands included).
//   MT = 0: v_mfma_f32_16x16x1f32, four blocks of 16 x 16: lane l supplies A(l / 16, l % 16) and B(l / 16, l % 16);
//           D(b, m, n) comes back in lane 16 (m / 4) + n, register 4 b + m % 4. A = x[l % 16] in every block: one
//           instruction advances 16 activation rows x 64 weight rows.
//   MT > 0: MT x v_mfma_f32_4x4x1f32, sixteen blocks of 4 x 4: lane l supplies A(l / 4, l % 4) and B(l / 4, l % 4);
//           D(b, m, n) comes back in lane 4 b + n, register m. Tile t takes A = x[4 t + l % 4]: 4 activation rows x
//           64 weight rows per instruction, and lane l collects its own row's results. At 9 cycles against 32.5 it
//           costs a quarter of the 16-row instruction for up to 4 rows.
template <int MT>
struct Tiles;

template <>
struct Tiles<0> {
    static constexpr int kRows = 16;
    v16f acc;
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    }
    __device__ __forceinline__ void step(const float *xs, int lane, const float y[32]) {
        const float *xr = xs + (lane & 15) * kXPitch;
        f32x4 xa[8];
#pragma unroll
        for (int q = 0; q < 8; q++) xa[q] = *reinterpret_cast<const f32x4 *>(xr + 4 * q);
#pragma unroll
        for (int e = 0; e < 32; e++) acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xa[e >> 2][e & 3], y[e], acc, 0, 0, 0);
    }
    __device__ __forceinline__ void store(float *res, int lane) const {  // res[m][row]
#pragma unroll
        for (int v = 0; v < 16; v++) res[(4 * (lane >> 4) + (v & 3)) * kRPitch + 16 * (v >> 2) + (lane & 15)] = acc[v];
    }
    // pp[m * ld + row] for m < mb, row < nrows
    __device__ __forceinline__ void store_global(float *pp, int64_t ld, int64_t mb, int64_t nrows, int lane) const {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = 4 * (lane >> 4) + (v & 3), row = 16 * (v >> 2) + (lane & 15);
            if (m < mb && row < nrows) pp[m * ld + row] = acc[v];
        }
    }
};

template <int MT>
struct Tiles {
    static constexpr int kRows = 4 * MT;
    v4f acc[MT];
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[t][v] = 0.0f;
    }
    __device__ __forceinline__ void step(const float *xs, int lane, const float y[32]) {
        f32x4 xa[MT][8];
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int q = 0; q < 8; q++)
                xa[t][q] = *reinterpret_cast<const f32x4 *>(xs + (4 * t + (lane & 3)) * kXPitch + 4 * q);
#pragma unroll
        for (int e = 0; e < 32; e++)
#pragma unroll
            for (int t = 0; t < MT; t++)
                acc[t] = __builtin_amdgcn_mfma_f32_4x4x1f32(xa[t][e >> 2][e & 3], y[e], acc[t], 0, 0, 0);
    }
    __device__ __forceinline__ void store(float *res, int lane) const {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) res[(4 * t + v) * kRPitch + lane] = acc[t][v];
    }
    __device__ __forceinline__ void store_global(float *pp, int64_t ld, int64_t mb, int64_t nrows, int lane) const {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                if (4 * t + v < mb && lane < nrows) pp[(4 * t + v) * ld + lane] = acc[t][v];
    }
};

// The same chains on the matrix cores, a pass of Tiles<MT>::kRows activation rows at a time, in ascending k from +0
// as the CPU kernel does. Activation rows past M repeat row M - 1; their results are dropped.
//
// Workgroup (blockIdx.x, blockIdx.y) covers rows 64 blockIdx.x .. +63 and chunks [cps blockIdx.y, + cps). A wave
// stages its chunk's weight images in LDS (loaded during its previous chunk) and each 32-wide group of activations
// (loaded a few groups ahead) in a 16 x 32 LDS tile that its lanes read back as A operands. With partial == null
// the workgroup covers every chunk and adds the chain results to `part` in chunk order in LDS; otherwise each
// chain result goes to partial[chunk][m][row] for sum_chunks_kernel.
template <int DT, bool ACC, int MT, int W>
__global__ __launch_bounds__(64 * W) void gemm_rows_mfma(const Planes p, const float *__restrict__ x,
                                                         float *__restrict__ c, float *__restrict__ partial, int64_t N,
                                                         int64_t row0, int64_t M, int64_t K, int64_t cps) {
    using I = Image<DT>;
    constexpr int XD = DT == kQ8 ? 1 : DT == kQ6K ? 2 : 4;  // activation groups in flight (larger images leave fewer registers)
    static_assert(16 * kRPitch * 4 <= 64 * I::kPitch, "chain results reuse the wave's image space");
    __shared__ __align__(16) uint8_t wsl[W][64 * I::kPitch];
    __shared__ __align__(16) float xsl[W][16 * kXPitch];
    const int lane = threadIdx.x & 63;
    const int cw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tm = threadIdx.x >> 6;  // summing role: activation rows tm + W j of the pass, weight row `lane`
    const int64_t rbase = (int64_t)blockIdx.x * 64;
    const int64_t r = rbase + lane;
    const int64_t nchunks = (K + 255) / 256;
    const int64_t cb = (int64_t)blockIdx.y * cps, ce = cb + cps < nchunks ? cb + cps : nchunks;
    uint8_t *ws = wsl[cw];
    float *xs = xsl[cw];
    const uint8_t *img = ws + lane * I::kPitch;
    constexpr int MP = Tiles<MT>::kRows;
    for (int64_t m0 = 0; m0 < M; m0 += MP) {
        const int64_t mb = (M - m0) < MP ? (M - m0) : MP;
        const float *xp[2];  // x piece P = 64 i + lane: activation row P / 8, floats 4 (P % 8) .. +3 of a group
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int P = 64 * i + lane, m = P >> 3;
            xp[i] = x + (m0 + (m < mb ? m : mb - 1)) * K + 4 * (P & 7);
        }
        f32x4 xg[XD][2];  // activations of the next XD groups; group g of every chunk uses slot g % XD
        constexpr int PR = 16 / W;
        float part[PR];
#pragma unroll
        for (int j = 0; j < PR; j++) part[j] = 0.0f;
        Stage<DT> st;
        if (cb + cw < ce) {
            st.load(p, row0, rbase, N, cb + cw, lane);
            const int64_t k0 = (cb + cw) * 256;
            const int ng0 = (int)(((K - k0) < 256 ? (K - k0) : 256) / 32);
#pragma unroll
            for (int g = 0; g < XD; g++)
                if (g < ng0) {
#pragma unroll
                    for (int i = 0; i < 2; i++) xg[g][i] = *reinterpret_cast<const f32x4 *>(xp[i] + k0 + 32 * g);
                }
        }
        for (int64_t c0 = cb; c0 < ce; c0 += W) {
            const int64_t pc = c0 + cw;
            if (pc < ce) {  // wave-uniform
                st.store(ws, lane);
                const uint32_t d6 = st.d6;
                const int64_t k0 = pc * 256;
                const int ngroups = (int)(((K - k0) < 256 ? (K - k0) : 256) / 32);
                const bool more = pc + W < ce;
                const int64_t kx = (pc + W) * 256;  // the wave's next chunk
                const int ngx = more ? (int)(((K - kx) < 256 ? (K - kx) : 256) / 32) : 0;
                Tiles<MT> tl;
                tl.zero();
                static_for<0, 8>([&](auto G) {
                    constexpr int gi = decltype(G)::value;
                    constexpr int sl = gi % XD;
                    if (gi < ngroups) {
                        __builtin_amdgcn_wave_barrier();
#pragma unroll
                        for (int i = 0; i < 2; i++) {
                            const int P = 64 * i + lane;
                            *reinterpret_cast<f32x4 *>(xs + (P >> 3) * kXPitch + 4 * (P & 7)) = xg[sl][i];
                        }
                        // the activations XD groups on, then (once a chunk) the next chunk's weights, are in flight
                        // during the arithmetic of the groups before them
                        constexpr int gn = gi + XD;
                        if (gn < ngroups || gn - ngroups < ngx) {
                            const int64_t kn = gn < ngroups ? k0 + 32 * gn : kx + 32 * (gn - ngroups);
#pragma unroll
                            for (int i = 0; i < 2; i++) xg[sl][i] = *reinterpret_cast<const f32x4 *>(xp[i] + kn);
                        }
                        if (gi == 0 && more) st.load(p, row0, rbase, N, pc + W, lane);
                        __builtin_amdgcn_wave_barrier();
                        Group<DT> g;
                        group_from_image<DT>(g, img, gi, d6);
                        float y[32];
                        g.decode(gi, y);
                        tl.step(xs, lane, y);
                    }
                });
                __builtin_amdgcn_wave_barrier();
                if (partial)
                    tl.store_global(partial + (pc * M + m0) * N + rbase, N, mb, N - rbase, lane);
                else
                    tl.store(reinterpret_cast<float *>(ws), lane);
            }
            if (!partial) {  // kernel-uniform
                __syncthreads();
                const int ng = (int)((ce - c0) < W ? (ce - c0) : W);
                for (int i = 0; i < ng; i++) {
                    const float *res = reinterpret_cast<const float *>(wsl[i]);
#pragma unroll
                    for (int j = 0; j < PR; j++)
                        if (tm + W * j < MP) part[j] = part[j] + res[(tm + W * j) * kRPitch + lane];
                }
                __syncthreads();
            }
        }
        if (!partial && r < N) {
#pragma unroll
            for (int j = 0; j < PR; j++)
                if (tm + W * j < mb) {
                    float *o = c + (m0 + tm + W * j) * N + r;
                    *o = ACC ? *o + part[j] : part[j];
                }
        }
    }
}

// c[i] (+)= (((0 + partial[0][i]) + partial[1][i]) + ...) over the chunks in order, i < M N.
template <bool ACC>
__global__ void sum_chunks_kernel(const float *__restrict__ partial, float *__restrict__ c, int64_t MN,
                                  int64_t nchunks) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < MN; i += (int64_t)gridDim.x * blockDim.x) {
        float part = 0.0f;
        for (int64_t ch = 0; ch < nchunks; ch += 8) {  // up to eight loads in flight, added in chunk order
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = ch + u < nchunks ? partial[(ch + u) * MN + i] : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (ch + u < nchunks) part = part + v[u];
        }
        c[i] = ACC ? c[i] + part : part;
    }
}


template <int DT, int MT, int W>
int run_tiles(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, float *partial,
              int64_t M, int64_t cps, int64_t nslices, bool acc) {
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)nslices), block(64 * W);
    if (acc)
        hipLaunchKernelGGL((gemm_rows_mfma<DT, true, MT, W>), grid, block, 0, ctx->stream, w->planes(), x, c, partial, N,
                           row0, M, w->K, cps);
    else
        hipLaunchKernelGGL((gemm_rows_mfma<DT, false, MT, W>), grid, block, 0, ctx->stream, w->planes(), x, c, partial,
                           N, row0, M, w->K, cps);
    return launch_check(ctx, "gemm_rows");
}

// Up to 4 activation rows: one 4-row tile; up to 8: two; more: passes of 16 rows.
template <int DT, int W>
int run_w(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, float *partial,
          int64_t M, int64_t cps, int64_t nslices, bool acc) {
    if (M <= 4) return run_tiles<DT, 1, W>(ctx, w, row0, N, x, c, partial, M, cps, nslices, acc);
    if (M <= 8) return run_tiles<DT, 2, W>(ctx, w, row0, N, x, c, partial, M, cps, nslices, acc);
    return run_tiles<DT, 0, W>(ctx, w, row0, N, x, c, partial, M, cps, nslices, acc);
}

template <int DT>
int run_dt(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, float *partial,
           int64_t M, int64_t cps, int64_t nslices, bool acc) {
    if (partial) return run_w<DT, kSplitWaves>(ctx, w, row0, N, x, c, partial, M, cps, nslices, acc);
    return run_w<DT, kStageWaves>(ctx, w, row0, N, x, c, partial, M, cps, nslices, acc);
}

}  // namespace

int launch_gemm_rows(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     int64_t M, bool acc) {
    if (N == 0 || M == 0) return TRHIP_OK;
    const int64_t K = w->K, nchunks = (K + 255) / 256, nrb = (N + 63) / 64;
    // One workgroup of kStageWaves waves per 64-row block covers all of its chunks when there are enough row blocks
    // to occupy the device; otherwise the chunks are split into slices of kSplitWaves chunks (about two workgroups
    // per CU in all) whose chain results are added in chunk order by sum_chunks_kernel.
    int64_t nslices = 1, cps = nchunks;
    if (nrb < 160 && nchunks > kSplitWaves) {
        const int64_t want = (512 + nrb - 1) / nrb;  // slices per row block for about 512 workgroups
        const int64_t maxs = (nchunks + kSplitWaves - 1) / kSplitWaves;
        nslices = want < maxs ? want : maxs;
        cps = (nchunks + nslices - 1) / nslices;
        cps = (cps + kSplitWaves - 1) / kSplitWaves * kSplitWaves;
        nslices = (nchunks + cps - 1) / cps;
    }
    const bool copy_x = reinterpret_cast<uintptr_t>(x) % 16 != 0;  // the kernel reads x 16 bytes at a time
    const size_t xbytes = copy_x ? ((size_t)(M * K) * sizeof(float) + 255) / 256 * 256 : 0;
    const size_t pbytes = nslices > 1 ? (size_t)(nchunks * M * N) * sizeof(float) : 0;
    int st = TRHIP_OK;
    uint8_t *ws = nullptr;
    if (xbytes + pbytes > 0) {
        ws = static_cast<uint8_t *>(workspace(ctx, xbytes + pbytes, &st));
        if (!ws) return st;
    }
    const float *xa = x;
    if (copy_x) {
        hipError_t e = hipMemcpyAsync(ws, x, (size_t)(M * K) * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "gemm_rows: align x");
        xa = reinterpret_cast<const float *>(ws);
    }
    float *partial = nslices > 1 ? reinterpret_cast<float *>(ws + xbytes) : nullptr;
    switch (w->dtype) {
    case kQ8: st = run_dt<kQ8>(ctx, w, row0, N, xa, c, partial, M, cps, nslices, acc); break;
    case kQ4: st = run_dt<kQ4>(ctx, w, row0, N, xa, c, partial, M, cps, nslices, acc); break;
    case kQ4K: st = run_dt<kQ4K>(ctx, w, row0, N, xa, c, partial, M, cps, nslices, acc); break;
    case kQ6K: st = run_dt<kQ6K>(ctx, w, row0, N, xa, c, partial, M, cps, nslices, acc); break;
    default: return fail(ctx, TRHIP_ERR_INVALID, "gemm_rows: bad dtype");
    }
    if (st != TRHIP_OK || !partial) return st;
    const int64_t MN = M * N;
    const unsigned blocks = (unsigned)((MN + 255) / 256 < 4096 ? (MN + 255) / 256 : 4096);
    if (acc)
        hipLaunchKernelGGL(sum_chunks_kernel<true>, dim3(blocks), dim3(256), 0, ctx->stream, partial, c, MN, nchunks);
    else
        hipLaunchKernelGGL(sum_chunks_kernel<false>, dim3(blocks), dim3(256), 0, ctx->stream, partial, c, MN, nchunks);
    return launch_check(ctx, "sum_chunks");
}

}  // namespace trhip
