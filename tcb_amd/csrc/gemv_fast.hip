// gemv_fast.hip -- decode GEMV (M == 1) in factored order: within the tolerance the reference allows a
// device GEMV (|a-b|/(1+|b|) <= 1e-5, 1e-4 for K-quants), not bit-identical to TR's CPU path.
//
// Per 32-element sub-block j with value y = s_j*q - m_j (tensor/quant.go:167-182):
//   sum_e y_e x_e = s_j * (sum_e q_e x_e) - m_j * (sum_e x_e)
// so the inner loop is one convert and one fused multiply-add per weight. The 16-element sums of x are the
// same for every row and are computed once per workgroup into LDS next to x.
//
// Every partial sum is combined in a fixed order inside one workgroup (LDS, then a fixed xor-butterfly),
// with no atomics, so the result depends only on the shape (the reference forbids atomic accumulation on
// this path, gpu/kernel_quant_gemv.go:14-16). Two kernels: gemv_fast_q4k (row-sliced, q4_k, the paragraphs
// above) and gemv_kl (K across lanes, fixed-point x on v_dot4, for q4_k, q6_k, q8_0 and q4_0; described below).
#include "trhip_internal.hpp"

#include <cstdio>
#include <cstdlib>

namespace trhip {
namespace {

// ---------------------------------------------------------------- q4_k
// Nibble pairs to floats: a byte holding 0..15, read as an OCP FP8 E4M3 value, is exactly q * 2^-9
// (subnormals below 8, the first binade above), so one v_cvt_pk_f32_fp8 converts two codes. The 2^9
// goes into the sub-block scale, which stays exact (a power of two).
__device__ __forceinline__ void fma_nib4(float &p, uint32_t nib4, float4 xv) {
    auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)nib4, false);  // bytes 0, 1
    auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)nib4, true);   // bytes 2, 3
    p = fmaf(lo[0], xv.x, p);
    p = fmaf(lo[1], xv.y, p);
    p = fmaf(hi[0], xv.z, p);
    p = fmaf(hi[1], xv.w, p);
}

// Eight lanes per row; lane (g, h) = (lane8 >> 1, lane8 & 1) owns the 16 qs bytes 32g + 16h .. +16 of
// every block: low nibbles are elements 16h..16h+15 of sub-block 2g, high nibbles the same elements of
// sub-block 2g+1. Each lane serves R rows (8 apart) with the same x, so a wave covers 8R rows and every x
// slice read from LDS feeds R rows. A workgroup is WAVES waves; with KS > 1 the waves form groups of KS on the
// same rows, each taking one KS-th of K (the parts meet in LDS and are added in part order), with KS = 1 each
// wave owns its rows' whole K. The 8 lanes of a row then add with a
// fixed xor-butterfly. x lives in LDS with a 16-byte pad per 256 bytes (the 8 slices a wave reads per step
// fall in distinct banks), its 16-element sums next to it. Weights are requested D blocks ahead, x one block
// ahead.
template <bool ACC, int D, int WAVES, int KS, int R>
__global__ __launch_bounds__(64 * WAVES) void gemv_fast_q4k(const Planes p, const float *__restrict__ x,
                                                            float *__restrict__ c, int64_t N, int64_t row0, int64_t K) {
    constexpr int THREADS = 64 * WAVES, ROWS = 8 * R * WAVES / KS;
    extern __shared__ float4 lds4[];
    __shared__ float part_lds[KS > 1 ? 64 * R * (WAVES / KS) * (KS - 1) : 1];
    const int nx4 = (int)(K / 4);
    float4 *xs = lds4;                                             // padded: nx4 + nx4/16 float4
    float *sx = reinterpret_cast<float *>(lds4 + nx4 + nx4 / 16);  // K/16 floats
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane8 = lane & 7, g = lane8 >> 1, hsel = lane8 & 1;
    const int rg = w / KS, part = w % KS;
    const int nb = (int)p.nb;
    const int nh = (nb + KS - 1) / KS;  // blocks per K part
    const int b0 = part * nh < nb ? part * nh : nb, b1 = b0 + nh < nb ? b0 + nh : nb;
    int64_t r[R];
    const uint4 *hp[R], *qp[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        r[i] = (int64_t)blockIdx.x * ROWS + 8 * R * rg + 8 * i + (lane >> 3);
        const int64_t row = row0 + (r[i] < N ? r[i] : N - 1);
        hp[i] = reinterpret_cast<const uint4 *>(p.aux) + row * nb;
        qp[i] = reinterpret_cast<const uint4 *>(p.qs) + row * nb * 8 + 4 * hsel + g;
    }
    uint4 H[D][R], Q[D][R];
#pragma unroll
    for (int s = 0; s < D; s++) {  // weights first: they come from HBM
        int b = b0 + s < b1 ? b0 + s : (b1 > b0 ? b1 - 1 : 0);
#pragma unroll
        for (int i = 0; i < R; i++) {
            H[s][i] = hp[i][b];
            Q[s][i] = qp[i][8 * b];
        }
    }
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int i = threadIdx.x; i < (int)(K / 16); i += THREADS) {
        float4 a = x4[4 * i], b = x4[4 * i + 1], cc = x4[4 * i + 2], dd = x4[4 * i + 3];
        float4 *o = xs + 4 * i + (i >> 2);  // padded index of 4i: 4i + (4i >> 4)
        o[0] = a;
        o[1] = b;
        o[2] = cc;
        o[3] = dd;
        sx[i] = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) + ((cc.x + cc.y) + (cc.z + cc.w)) +
                ((dd.x + dd.y) + (dd.z + dd.w));
    }
    __syncthreads();
    const int k0 = (2 * g) & 3, k1 = (2 * g + 1) & 3;
    // x of elements 256b + 64g + 16h + 4c (+32 for the high nibbles): float4 64b + 16g + 4h + c, padded
    // by (64b + 16g + 4h + c) >> 4 = 4b + g
    const float4 *xg = xs + 17 * g + 4 * hsel;
    const float *sxg = sx + 4 * g + hsel;
    float4 XL[4], XH[4];
    {
        const float4 *xb = xg + 68 * (b0 < b1 ? b0 : 0);
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            XL[cc] = xb[cc];
            XH[cc] = xb[8 + cc];
        }
    }
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; i++) acc[i] = 0.0f;
    for (int bb = b0; bb < b1; bb += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            const int b = bb + s;
            uint4 h[R], q[R];
            const int nx = b + D < b1 ? b + D : b1 - 1;
#pragma unroll
            for (int i = 0; i < R; i++) {
                h[i] = H[s][i];
                q[i] = Q[s][i];
                H[s][i] = hp[i][nx];
                Q[s][i] = qp[i][8 * nx];
            }
            const float4 *xn = xg + 68 * (b + 1 < b1 ? b + 1 : b);
            float4 NL[4], NH[4];
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                NL[cc] = xn[cc];
                NH[cc] = xn[8 + cc];
            }
            if (b < b1) {  // wave-uniform
                const float *sxb = sxg + 16 * b;
                const float sl = sxb[0], shx = sxb[2];
#pragma unroll
                for (int i = 0; i < R; i++) {
                    float d = f16_to_f32((uint16_t)(h[i].x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(h[i].x >> 16));
                    uint32_t sc_lo, sc_hi, m_lo, m_hi;
                    q4k_scales(h[i].y, h[i].z, h[i].w, sc_lo, sc_hi, m_lo, m_hi);
                    const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
                    const float d9 = d * 512.0f;  // undoes the 2^-9 of the fp8 reading
                    const float s0 = d9 * ubyte_f(scw, k0), n0 = -(dmin * ubyte_f(mw, k0));
                    const float s1 = d9 * ubyte_f(scw, k1), n1 = -(dmin * ubyte_f(mw, k1));
                    const uint32_t qw[4] = {q[i].x, q[i].y, q[i].z, q[i].w};
                    float pl0 = 0.0f, pl1 = 0.0f, ph0 = 0.0f, ph1 = 0.0f;
#pragma unroll
                    for (int cc = 0; cc < 4; cc++) {
                        const uint32_t lo = qw[cc] & 0x0F0F0F0Fu, hi = (qw[cc] >> 4) & 0x0F0F0F0Fu;
                        float &pl = (cc & 1) ? pl1 : pl0;
                        float &ph = (cc & 1) ? ph1 : ph0;
                        fma_nib4(pl, lo, XL[cc]);
                        fma_nib4(ph, hi, XH[cc]);
                    }
                    acc[i] = fmaf(s0, pl0 + pl1, acc[i]);
                    acc[i] = fmaf(n0, sl, acc[i]);
                    acc[i] = fmaf(s1, ph0 + ph1, acc[i]);
                    acc[i] = fmaf(n1, shx, acc[i]);
                }
            }
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                XL[cc] = NL[cc];
                XH[cc] = NH[cc];
            }
        }
    }
    if (KS > 1) {  // parts 1..KS-1 hand their sums to part 0, which adds them in part order
        constexpr int RG = WAVES / KS;
        if (part) {
#pragma unroll
            for (int i = 0; i < R; i++) part_lds[64 * (((part - 1) * RG + rg) * R + i) + lane] = acc[i];
        }
        __syncthreads();
        if (part) return;
#pragma unroll
        for (int q = 1; q < KS; q++)
#pragma unroll
            for (int i = 0; i < R; i++) acc[i] = acc[i] + part_lds[64 * (((q - 1) * RG + rg) * R + i) + lane];
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
        float a = acc[i];
        a += __shfl_xor(a, 1);
        a += __shfl_xor(a, 2);
        a += __shfl_xor(a, 4);
        if (lane8 == 0 && r[i] < N) c[r[i]] = ACC ? c[r[i]] + a : a;
    }
}

// Fixed-order sum over the 64 lanes of eight values per lane (one per row), all in VALU lane permutes: two
// transpose levels with v_permlane32_swap / v_permlane16_swap (each swap leaves, in the two registers, the
// halves a lane must add), a third through DPP row_ror:8, then three DPP levels inside each group of 8 lanes
// (row_half_mirror, quad_perm [2,3,0,1], quad_perm [1,0,3,2]). Lane l ends with the full sum of row l >> 3.
// The swap results pass through opaque(): read as floats straight from the builtin's pair, this compiler
// folds the two halves into one register (v_add_f32 vN, vN, vN).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_sum8(float v[8], int lane) {
    float u[4], t[2];
#pragma unroll
    for (int i = 0; i < 4; i++) {  // lanes 0-31 keep row i, lanes 32-63 row i + 4
        const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v[i]),
                                                        __builtin_bit_cast(unsigned, v[i + 4]), false, false);
        u[i] = __builtin_bit_cast(float, opaque(r[0])) + __builtin_bit_cast(float, opaque(r[1]));
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {  // lane bit 4 selects row +2
        const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, u[i]),
                                                        __builtin_bit_cast(unsigned, u[i + 2]), false, false);
        t[i] = __builtin_bit_cast(float, opaque(r[0])) + __builtin_bit_cast(float, opaque(r[1]));
    }
    const bool b3 = lane & 8;  // lane bit 3 selects row +1
    const float keep = b3 ? t[1] : t[0], send = b3 ? t[0] : t[1];
    float a = keep + dpp_f<0x128>(send);  // row_ror:8 is lane ^ 8 inside 16 lanes
    a = a + dpp_f<0x141>(a);              // row_half_mirror: lane ^ 7 inside 8 lanes
    a = a + dpp_f<0x4E>(a);               // quad_perm [2,3,0,1]
    a = a + dpp_f<0xB1>(a);               // quad_perm [1,0,3,2]
    return a;
}

// Fixed-point x for v_dot4_i32_i8: within a 32-element half, X = rint(x * 2^(23-e)) with e from grid_exp, so
// |X| <= 2^23 * 127/128, split into signed bytes X = d2*2^16 + d1*2^8 + d0 (d0, d1 in [-128, 127], |d2| <= 127).
// x4_digits packs the digits of four consecutive elements into three dwords (digit t of element k in byte k of
// dword t); one unit of X weighs 2^(e-23).
// The digits come from U = X + 0x808080, which lies in [0, 2^24): byte t of U is d_t + 128 (the digits above are
// the only ones in [-128, 127] with X = d0 + 256 d1 + 65536 d2), so four v_perm_b32 gathers plus one per digit word
// and an xor of the 0x80 offsets pack them.
__device__ __forceinline__ void x4_digits(const float *xv, int e, uint32_t out[3]) {
    uint32_t u[4];
#pragma unroll
    for (int k = 0; k < 4; k++) u[k] = (uint32_t)((int)rintf(ldexpf(xv[k], 23 - e)) + 0x808080);
    // __builtin_amdgcn_perm(s0, s1, sel): byte i of the result is byte sel_i of the eight bytes s1 (0..3), s0 (4..7)
    const uint32_t a = __builtin_amdgcn_perm(u[1], u[0], 0x05010400u);  // u0.0 u1.0 u0.1 u1.1
    const uint32_t b = __builtin_amdgcn_perm(u[3], u[2], 0x05010400u);  // u2.0 u3.0 u2.1 u3.1
    const uint32_t c = __builtin_amdgcn_perm(u[1], u[0], 0x07030602u);  // u0.2 u1.2 u0.3 u1.3
    const uint32_t d = __builtin_amdgcn_perm(u[3], u[2], 0x07030602u);  // u2.2 u3.2 u2.3 u3.3
    out[0] = __builtin_amdgcn_perm(b, a, 0x05040100u) ^ 0x80808080u;
    out[1] = __builtin_amdgcn_perm(b, a, 0x07060302u) ^ 0x80808080u;
    out[2] = __builtin_amdgcn_perm(d, c, 0x05040100u) ^ 0x80808080u;
}

// Exponent of a half's grid: m = f * 2^e with f in [0.5, 1) (0 gives e = 0), raised by one when f > 127/128, so
// that |x| * 2^(23-e) <= 2^23 * 127/128 and the top digit stays a signed byte.
__device__ __forceinline__ int grid_exp(float m) {
    int e = 0;
    const float f = frexpf(m, &e);
    return f > 127.0f / 128.0f ? e + 1 : e;
}

// q4_k, K across lanes. A K part is up to 16 blocks; lane l of a wave owns quarter g = l & 3 of block l >> 2 of
// its part: qs bytes 32g .. 32g+31 (the low nibbles are sub-block 2g, the high nibbles sub-block 2g+1), i.e. the
// 64 contiguous elements 256b + 64g .. +63. Their x stays in registers for the whole kernel as fixed-point digits
// (x4_digits), so the products with the 4-bit codes are exact integer dot products (v_dot4_i32_i8, one per digit
// and four codes) and only the per-sub-block sums are rounded:
//   sum_e y_e x_e = s_j * 2^(e-23) * (sum_e q_e X_e) - m_j * (sum_e x_e).
// The fixed-point x is exact to 2^-23 of the largest |x| of its 32-element half; a lane whose x holds Inf or NaN
// (or whose x sums overflow) takes float products of the dequantized values instead (IEEE propagation).
//
// A wave streams whole rows: per row, 64 lanes read 2 KB of qs (32 contiguous bytes each) and the block headers,
// and each lane leaves one partial; eight rows' partials meet in lane_sum8. A row group (the KS waves that
// share rows) takes rows gw, gw + G, gw + 2G, ... (G row groups in the grid, at most RPW rows each, all in
// straight-line code so the loads' wait counts stay exact); slots past a group's last row re-read that row
// (its own, cached) and are not stored. With KS > 1 the parts 1..KS-1 hand their row sums through LDS to
// part 0, which adds them in part order. The RG row groups of a part share x: each loads and digitizes 16 / RG
// of the 16 four-element columns, through LDS. Weights are requested PD rows ahead, after x.
//
// q8_0 / q4_0 (32-element blocks, y = d*q and y = d*(q - 8), tensor/quant.go:139-155) use the same lanes, x
// digits and row streaming: lane l owns blocks 2l and 2l + 1 of its part (up to 128 blocks), which are the same
// 64 contiguous elements, one block per 32-element half. q8_0: the codes are signed bytes, four per v_dot4;
// q4_0: byte j of a block holds elements j (low nibble) and j + 16 (high nibble), so the low nibbles meet digit
// words 0..3 of the half and the high nibbles words 4..7. Per block, sum_e y_e x_e = d * 2^(e-23) * sum_e q_e X_e
// (q8_0) or d * (2^(e-23) * sum_e q_e X_e - 8 * sum_e x_e) (q4_0).
template <int DT>
struct KlRow;  // one row slot: the bytes a lane reads for its 64 elements

template <>
struct KlRow<kQ4K> {
    uint4 h, q0, q1;
};
template <>
struct KlRow<kQ8> {
    uint4 q[4];
    uint32_t d;  // the two blocks' fp16 scales
};
template <>
struct KlRow<kQ4> {
    uint4 q0, q1;
    uint32_t d;
};
template <>
struct KlRow<kQ6K> {  // ql pieces t at 32t + 16n, qh pieces at 16t + 8n, the lane's four scales, d
    uint4 ql[4];
    uint2 qh[4];
    uint32_t sc, d;
};

// SWI: the store holds 2N rows, [gate | up] (a merged gate_up layer), and c receives silu(g_i) * u_i for i < N.
// Slots then alternate gate row i and up row N + i of the same pair; a row's sum does not depend on its slot
// (lane_sum8 pairs the same lanes for every slot), so the outputs are the unfused GEMV's sums gated exactly as
// swiglu_kernel gates them.
// SKIP: the grid has more row groups than RPW-row groups need, so a group's last slots may lie past its rows; they
// still load (a re-read of the last row, which keeps every wait count fixed) but skip the arithmetic
// IO: TRHIP_F32, or TRHIP_F16 / TRHIP_BF16 for 16-bit x read and 16-bit c written directly (widened exactly and
// rounded once, as the typed entry point's staged path does; not with SWI).
template <int DT, bool ACC, int WAVES, int KS, int PD, int RPW, bool SWI = false, bool SKIP = false, int IO = TRHIP_F32>
__global__ __launch_bounds__(64 * WAVES) void gemv_kl(const Planes p, const void *__restrict__ xv,
                                                      void *__restrict__ cv, int64_t N, int64_t row0) {
    static_assert(IO == TRHIP_F32 || !SWI, "the gated output is fp32");
    static_assert(!(SWI && ACC), "the gated output is set, not accumulated");
    static_assert(!SWI || RPW % 2 == 0, "slots come in gate / up pairs");
    constexpr int RG = WAVES / KS;
    static_assert(16 % RG == 0, "the row groups of a part split the 16 columns of x evenly");
    static_assert(RPW % PD == 0, "rows are consumed PD at a time from a ring of PD slots");
    constexpr int CPW = 16 / RG;
    __shared__ float part_lds[2][KS > 1 ? (KS - 1) * RG * 8 : 1];
    __shared__ uint32_t xd_lds[KS][16][3][64];
    __shared__ float4 xp_lds[KS][RG][64];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = w / KS, part = w % KS;
    const int nb = (int)p.nb;
    constexpr bool K4 = DT == kQ4K || DT == kQ6K;  // 256-element blocks, four lanes per block
    // blocks per part (even for q8_0 / q4_0: the launcher requires an even block count)
    const int bpp = K4 ? (nb + KS - 1) / KS : ((nb + KS - 1) / KS + 1) / 2 * 2;
    const int pb0 = part * bpp, pb1 = pb0 + bpp < nb ? pb0 + bpp : nb;
    const int g = lane & 3, b = pb0 + (K4 ? (lane >> 2) : 2 * lane);
    const bool active = b < pb1;
    const int bc = active ? b : (pb0 < nb ? pb0 : (K4 ? nb - 1 : nb - 2));  // inactive lanes read valid blocks
    // this lane's x, four elements at a time from element xe0 (widened exactly when 16-bit)
    const int64_t xe0 = K4 ? 256 * (int64_t)bc + 64 * g : 32 * (int64_t)bc;
    auto x4 = [&](int i) -> float4 {
        if constexpr (IO == TRHIP_F32) {
            return reinterpret_cast<const float4 *>(static_cast<const float *>(xv) + xe0)[i];
        } else {
            const uint2 h = reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(xv) + xe0)[i];
            return make_float4(h16_to_f32(h.x & 0xFFFFu, IO), h16_to_f32(h.x >> 16, IO), h16_to_f32(h.y & 0xFFFFu, IO),
                               h16_to_f32(h.y >> 16, IO));
        }
    };
    float *c = static_cast<float *>(cv);  // (IO == TRHIP_F32)
    // issue order: this wave's columns of x (cache-resident), then the first PD rows, so that waiting for x
    // leaves the rows in flight
    float4 xraw[CPW];
#pragma unroll
    for (int i = 0; i < CPW; i++) xraw[i] = x4(rg * CPW + i);
    const int k0 = (2 * g) & 3, k1 = k0 + 1;
    // q4_k: header of the lane's block, and qs 16-byte pieces g and g + 4 of it; q8_0 / q4_0: the two blocks'
    // codes (64 / 32 contiguous bytes) and their two fp16 scales (one aligned dword)
    // Loads address a row's planes from a wave-uniform row base plus a fixed 32-bit byte offset per lane, so the
    // per-row address arithmetic is mostly scalar (two vector adds per row remain, from four).
    // q6_k: elements 64g .. 64g+63 of the block are 32-element groups k4 = 2 (g & 1) and + 1 of half n = g >> 1;
    // the repacked ql bytes of (t, k4 & 1, l) sit at 32t + 16n + 8 (k4 & 1) + l (low nibbles for k4 < 2), the qh
    // bytes of (t, l) at 16t + 8n + l (bits 2 k4), the scales of the four 16-element quarters at 8n + 4 (g & 1)
    const int n6 = g >> 1;
    const uint32_t o_qs = K4 ? 128u * bc + 16u * (DT == kQ4K ? g : n6) : (uint32_t)qs_bytes(DT) * bc;
    const uint32_t o_aux = DT == kQ4K ? 16u * bc : 64u * bc + 8u * n6;
    const uint32_t o_sc = 16u * bc + 8u * n6 + 4u * (g & 1);
    const uint32_t o_d = 2u * bc;  // q8_0 / q4_0 (bc even): the aligned dword of blocks bc, bc + 1
    auto at = [](const void *base, int64_t off, uint32_t lane_off) {
        return reinterpret_cast<const uint8_t *>(base) + off + lane_off;
    };
    auto load_row = [&](KlRow<DT> &rw, int64_t row) {
        const int64_t rb = row * nb;  // blocks before the row
        if constexpr (DT == kQ4K) {
            rw.h = *reinterpret_cast<const uint4 *>(at(p.aux, rb * 16, o_aux));
            rw.q0 = *reinterpret_cast<const uint4 *>(at(p.qs, rb * 128, o_qs));
            rw.q1 = *reinterpret_cast<const uint4 *>(at(p.qs, rb * 128, o_qs + 64));
        } else if constexpr (DT == kQ6K) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                rw.ql[t] = *reinterpret_cast<const uint4 *>(at(p.qs, rb * 128, o_qs + 32 * t));
                rw.qh[t] = *reinterpret_cast<const uint2 *>(at(p.aux, rb * 64, o_aux + 16 * t));
            }
            rw.sc = *reinterpret_cast<const uint32_t *>(at(p.sc, rb * 16, o_sc));
            rw.d = *reinterpret_cast<const uint16_t *>(at(p.d, rb * 2, o_d));
        } else if constexpr (DT == kQ8) {
#pragma unroll
            for (int i = 0; i < 4; i++) rw.q[i] = *reinterpret_cast<const uint4 *>(at(p.qs, rb * 32, o_qs + 16 * i));
            rw.d = *reinterpret_cast<const uint32_t *>(at(p.d, rb * 2, o_d));
        } else {
            rw.q0 = *reinterpret_cast<const uint4 *>(at(p.qs, rb * 16, o_qs));
            rw.q1 = *reinterpret_cast<const uint4 *>(at(p.qs, rb * 16, o_qs + 16));
            rw.d = *reinterpret_cast<const uint32_t *>(at(p.d, rb * 2, o_d));
        }
    };
    // row counts fit 32 bits (the launcher checks), so the uniform row arithmetic stays 32-bit. Without SWI slot i is
    // output row gw + i G; with SWI, slots 2j and 2j + 1 are gate row gw + j G and up row N + gw + j G
    const uint32_t G = gridDim.x * RG, gw = blockIdx.x * RG + rg, n32 = (uint32_t)N;
    const uint32_t nv = gw < n32 ? (n32 - 1 - gw) / G + 1 : 0;                 // outputs of this row group
    const uint32_t last = nv > 0 ? gw + (nv - 1) * G : gw - (gw / n32) * n32;  // what slots past them re-read
    auto row_of = [&](int i) {
        if constexpr (SWI) {
            const uint32_t j = (uint32_t)i >> 1, o = j < nv ? gw + j * G : last;
            return row0 + (int64_t)o + ((i & 1) ? N : 0);
        } else {
            return row0 + (int64_t)((uint32_t)i < nv ? gw + (uint32_t)i * G : last);
        }
    };
    KlRow<DT> R[PD];
#pragma unroll
    for (int s = 0; s < PD; s++) load_row(R[s], row_of(s));
    __builtin_amdgcn_sched_barrier(0);
    // per-wave partial sums and maxima of its columns' halves meet in LDS (added in wave order); then each wave
    // turns its columns into digits for all 64 lanes, which every wave of the part reads back
    int xd[2][8][3];
    int ex[2];  // one unit of X weighs 2^ex (applied last, so subnormal x keeps its value)
    float sxl = 0.0f, sxh = 0.0f;
    {
        // half (hf) of each column: fixed for RG = 1 (one wave holds all 16 columns); for RG > 1 a wave's CPW <= 8
        // columns lie in one half, so one running sum and maximum serve and are placed in that half at the end
        float ps[2] = {0.0f, 0.0f}, pm[2] = {0.0f, 0.0f}, xc[CPW * 4];
#pragma unroll
        for (int i = 0; i < CPW; i++) {
            const float4 t = xraw[i];
            const float e4[4] = {active ? t.x : 0.0f, active ? t.y : 0.0f, active ? t.z : 0.0f, active ? t.w : 0.0f};
            const int hf = RG == 1 ? i >> 3 : 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                xc[4 * i + k] = e4[k];
                ps[hf] += e4[k];
                pm[hf] = fmaxf(pm[hf], fabsf(e4[k]));
            }
        }
        if (RG > 1 && (rg * CPW) >= 8) {  // wave-uniform
            ps[1] = ps[0];
            pm[1] = pm[0];
            ps[0] = 0.0f;
            pm[0] = 0.0f;
        }
        xp_lds[part][rg][lane] = make_float4(ps[0], ps[1], pm[0], pm[1]);
        __syncthreads();
        float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
        for (int q = 0; q < RG; q++) {
            const float4 t = xp_lds[part][q][lane];
            sxl += t.x;
            sxh += t.y;
            m0 = fmaxf(m0, t.z);
            m1 = fmaxf(m1, t.w);
        }
        const int e0 = grid_exp(m0), e1 = grid_exp(m1);
        ex[0] = e0 - 23;
        ex[1] = e1 - 23;
#pragma unroll
        for (int i = 0; i < CPW; i++) {
            const int col = rg * CPW + i;
            uint32_t dg[3];
            x4_digits(xc + 4 * i, col < 8 ? e0 : e1, dg);
#pragma unroll
            for (int t = 0; t < 3; t++) xd_lds[part][col][t][lane] = dg[t];
        }
        __syncthreads();
#pragma unroll
        for (int col = 0; col < 16; col++)
#pragma unroll
            for (int t = 0; t < 3; t++) xd[col >> 3][col & 7][t] = (int)xd_lds[part][col][t][lane];
    }
    const bool fin = __builtin_isfinite(sxl) && __builtin_isfinite(sxh);  // false also when a finite sum overflows
    // q6_k: every 16-element quarter's chains start at -32 * (its digit sum), so that they hold sum (q - 32) X
    int c6[4][3];
    if constexpr (DT == kQ6K) {
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int t = 0; t < 3; t++) {
                int sdg = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) sdg = __builtin_amdgcn_sdot4(0x01010101, xd[q >> 1][4 * (q & 1) + k][t], sdg, false);
                c6[q][t] = -32 * sdg;
            }
    }
    // q4_k: the high nibbles stay in place as the signed bytes (16 q - 128) = (w ^ 0x80) & 0xF0 (one v_bitop3), so
    // their chains start at 128 times the high half's digit sums and end at exactly 16 sum q X; the lane's scale
    // and min bytes are shifted to bytes 0 and 1 (shifts sa, sy, sm below) from header words chosen by g
    int hc[3] = {0, 0, 0};
    if constexpr (DT == kQ4K) {
#pragma unroll
        for (int t = 0; t < 3; t++) {
            int sdg = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) sdg = __builtin_amdgcn_sdot4(0x01010101, xd[1][k][t], sdg, false);
            hc[t] = 128 * sdg;
        }
    }
    const uint32_t sa = 16u * (g & 1), sy = sa + (g < 2 ? 0u : 2u), sm = sa + (g < 2 ? 0u : 4u);
    const int exh = ex[1] - 4;  // the high half's sums are 16 times too large
#pragma unroll
    for (int i0 = 0; i0 < RPW; i0 += 8) {
        float v[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const int slot = s % PD;
            const KlRow<DT> rw = R[slot];
            // (SKIP) a slot past the group's last row skips the arithmetic: its sum is not stored
            const bool used = !SKIP || (uint32_t)(SWI ? (i0 + s) >> 1 : i0 + s) < nv;  // wave-uniform
            float a = 0.0f;
            if (used) {
            if constexpr (DT == kQ6K) {
            const float d6 = f16_to_f32((uint16_t)(rw.d & 0xFFFF));
            const int sh = 4 * (g & 1);  // this lane's nibble and its qh bit pair base
            uint32_t code[2][8];  // [k4 & 1][word]: codes 0..63 of elements 4 word .. +3 of the group
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t lw[4] = {rw.ql[t].x, rw.ql[t].y, rw.ql[t].z, rw.ql[t].w};
                const uint32_t hw[2] = {rw.qh[t].x, rw.qh[t].y};
#pragma unroll
                for (int kk = 0; kk < 2; kk++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const uint32_t nib = (lw[2 * kk + j] >> sh) & 0x0F0F0F0Fu;
                        const uint32_t hi2 = ((hw[j] >> (sh + 2 * kk)) & 0x03030303u) << 4;
                        code[kk][2 * t + j] = nib | hi2;
                    }
            }
            float pq[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int cw0 = (int)code[q >> 1][4 * (q & 1)];
                int l0 = sdot4_from(cw0, xd[q >> 1][4 * (q & 1)][0], c6[q][0]);
                int l1 = sdot4_from(cw0, xd[q >> 1][4 * (q & 1)][1], c6[q][1]);
                int l2 = sdot4_from(cw0, xd[q >> 1][4 * (q & 1)][2], c6[q][2]);
#pragma unroll
                for (int k = 1; k < 4; k++) {
                    const int cw = (int)code[q >> 1][4 * (q & 1) + k];
                    l0 = __builtin_amdgcn_sdot4(cw, xd[q >> 1][4 * (q & 1) + k][0], l0, false);
                    l1 = __builtin_amdgcn_sdot4(cw, xd[q >> 1][4 * (q & 1) + k][1], l1, false);
                    l2 = __builtin_amdgcn_sdot4(cw, xd[q >> 1][4 * (q & 1) + k][2], l2, false);
                }
                pq[q] = fmaf((float)l2, 65536.0f, fmaf((float)l1, 256.0f, (float)l0));
            }
            const float s0 = (float)(int8_t)(rw.sc & 0xFF), s1 = (float)(int8_t)((rw.sc >> 8) & 0xFF);
            const float s2 = (float)(int8_t)((rw.sc >> 16) & 0xFF), s3 = (float)(int8_t)(rw.sc >> 24);
            a = ldexpf(d6 * fmaf(s1, pq[1], s0 * pq[0]), ex[0]) + ldexpf(d6 * fmaf(s3, pq[3], s2 * pq[2]), ex[1]);
            if (!fin) {  // Inf or NaN in this lane's x: dequantized values times x in float
                a = 0.0f;
#pragma unroll
                for (int kk = 0; kk < 2; kk++)
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const float4 xq = x4(8 * kk + k);
                        const float xs[4] = {xq.x, xq.y, xq.z, xq.w};
                        const float ds = d6 * (float)(int8_t)((rw.sc >> (8 * (2 * kk + (k >> 2)))) & 0xFF);
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            a = fmaf(ds * (ubyte_f(code[kk][k], e) - 32.0f), xs[e], a);  // fl(fl(d*sc)*(q-32))
                    }
            }
            } else if constexpr (DT == kQ4K) {
            const uint4 h = rw.h, q0 = rw.q0, q1 = rw.q1;
            const float d = f16_to_f32((uint16_t)(h.x & 0xFFFF)), dmin = f16_to_f32((uint16_t)(h.x >> 16));
            // scale and min of sub-blocks 2g and 2g + 1 unpacked into bytes 0 and 1 (tensor/quant.go:158-163): g < 2
            // keeps six bits of scale word y / z, g >= 2 four bits of word w and the top two of y / z
            const uint32_t xs = (g < 2 ? h.y : h.w) >> sa, xm = (g < 2 ? h.z : h.w) >> sm;
            const uint32_t sc2 = (xs & 0x0F0Fu) | ((h.y >> sy) & 0x3030u), m2 = (xm & 0x0F0Fu) | ((h.z >> sy) & 0x3030u);
            const float sc0 = ubyte_f(sc2, 0), sc1 = ubyte_f(sc2, 1), m0 = ubyte_f(m2, 0), m1 = ubyte_f(m2, 1);
            const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            int l0, l1, l2, h0, h1, h2;
            {
                const int lo = (int)(qw[0] & 0x0F0F0F0Fu), hi = (int)((qw[0] ^ 0x80808080u) & 0xF0F0F0F0u);
                l0 = sdot4_zero(lo, xd[0][0][0]);
                l1 = sdot4_zero(lo, xd[0][0][1]);
                l2 = sdot4_zero(lo, xd[0][0][2]);
                h0 = sdot4_from(hi, xd[1][0][0], hc[0]);
                h1 = sdot4_from(hi, xd[1][0][1], hc[1]);
                h2 = sdot4_from(hi, xd[1][0][2], hc[2]);
            }
#pragma unroll
            for (int k = 1; k < 8; k++) {
                const int lo = (int)(qw[k] & 0x0F0F0F0Fu), hi = (int)((qw[k] ^ 0x80808080u) & 0xF0F0F0F0u);
                l0 = __builtin_amdgcn_sdot4(lo, xd[0][k][0], l0, false);
                l1 = __builtin_amdgcn_sdot4(lo, xd[0][k][1], l1, false);
                l2 = __builtin_amdgcn_sdot4(lo, xd[0][k][2], l2, false);
                h0 = __builtin_amdgcn_sdot4(hi, xd[1][k][0], h0, false);
                h1 = __builtin_amdgcn_sdot4(hi, xd[1][k][1], h1, false);
                h2 = __builtin_amdgcn_sdot4(hi, xd[1][k][2], h2, false);
            }
            // |l1| * 256 + |l0| < 2^24, so the first two digits add exactly, in 32-bit integers as in float (the high
            // half's, 16 times as large, too: a multiple of 16 below 2^28)
            const float pl = fmaf((float)l2, 65536.0f, (float)(l1 * 256 + l0));
            const float ph = fmaf((float)h2, 65536.0f, (float)(h1 * 256 + h0));
            // d and dmin are applied before the 2^e scaling, so no partial overflows ahead of the sum itself
            const float s0 = d * sc0, n0 = -(dmin * m0), s1 = d * sc1, n1 = -(dmin * m1);
            a = ldexpf(s0 * pl, ex[0]);
            a = fmaf(n0, sxl, a);
            a = a + ldexpf(s1 * ph, exh);
            a = fmaf(n1, sxh, a);
            if (!fin) {  // Inf or NaN in this lane's x: dequantized values times x in float
                a = 0.0f;
                auto part = [&](int k) {
                    const float4 xl = x4(k), xh = x4(8 + k);
                    const uint32_t lo = qw[k] & 0x0F0F0F0Fu, hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
                    const float xlv[4] = {xl.x, xl.y, xl.z, xl.w}, xhv[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        a = fmaf(fmaf(s0, ubyte_f(lo, t), n0), xlv[t], a);
                        a = fmaf(fmaf(s1, ubyte_f(hi, t), n1), xhv[t], a);
                    }
                };
                if constexpr (IO == TRHIP_F32) {
#pragma unroll
                    for (int k = 0; k < 8; k++) part(k);
                } else {  // rolled: widening x here would otherwise grow every row slot's code past what unrolls
#pragma unroll 1
                    for (int k = 0; k < 8; k++) part(k);
                }
            }
            } else {
            // q8_0: 16 code words, 8 per block; q4_0: 8 words, 4 per block (low nibbles then high nibbles)
            const float d0 = f16_to_f32((uint16_t)(rw.d & 0xFFFF)), d1 = f16_to_f32((uint16_t)(rw.d >> 16));
            int acc8[2][3];
            uint32_t qw[16];
            if constexpr (DT == kQ8) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    qw[4 * i] = rw.q[i].x;
                    qw[4 * i + 1] = rw.q[i].y;
                    qw[4 * i + 2] = rw.q[i].z;
                    qw[4 * i + 3] = rw.q[i].w;
                }
#pragma unroll
                for (int hf = 0; hf < 2; hf++)
#pragma unroll
                    for (int k = 0; k < 8; k++)
#pragma unroll
                        for (int t = 0; t < 3; t++)
                            acc8[hf][t] = k == 0 ? sdot4_zero((int)qw[8 * hf], xd[hf][0][t])
                                                 : __builtin_amdgcn_sdot4((int)qw[8 * hf + k], xd[hf][k][t], acc8[hf][t], false);
            } else {
                const uint32_t w8[8] = {rw.q0.x, rw.q0.y, rw.q0.z, rw.q0.w, rw.q1.x, rw.q1.y, rw.q1.z, rw.q1.w};
#pragma unroll
                for (int hf = 0; hf < 2; hf++)
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t wd = w8[4 * hf + k];
                        qw[8 * hf + k] = wd & 0x0F0F0F0Fu;             // elements 4k .. 4k+3
                        qw[8 * hf + 4 + k] = (wd >> 4) & 0x0F0F0F0Fu;  // elements 16 + 4k ..
                    }
#pragma unroll
                for (int hf = 0; hf < 2; hf++)
#pragma unroll
                    for (int k = 0; k < 8; k++)
#pragma unroll
                        for (int t = 0; t < 3; t++)
                            acc8[hf][t] = k == 0 ? sdot4_zero((int)qw[8 * hf], xd[hf][0][t])
                                                 : __builtin_amdgcn_sdot4((int)qw[8 * hf + k], xd[hf][k][t], acc8[hf][t], false);
            }
            const float pl = fmaf((float)acc8[0][2], 65536.0f, fmaf((float)acc8[0][1], 256.0f, (float)acc8[0][0]));
            const float ph = fmaf((float)acc8[1][2], 65536.0f, fmaf((float)acc8[1][1], 256.0f, (float)acc8[1][0]));
            if constexpr (DT == kQ8) {
                a = d0 * ldexpf(pl, ex[0]) + d1 * ldexpf(ph, ex[1]);
            } else {
                a = d0 * fmaf(-8.0f, sxl, ldexpf(pl, ex[0])) + d1 * fmaf(-8.0f, sxh, ldexpf(ph, ex[1]));
            }
            if (!fin) {  // Inf or NaN in this lane's x: dequantized values times x in float
                a = 0.0f;
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const float dd = hf ? d1 : d0;
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        const float4 xq = x4(8 * hf + k);
                        const float xs[4] = {xq.x, xq.y, xq.z, xq.w};
                        const uint32_t wq = qw[8 * hf + k];
#pragma unroll
                        for (int t = 0; t < 4; t++) {
                            const float q = DT == kQ8 ? (float)(int8_t)((wq >> (8 * t)) & 0xFF)
                                                      : ubyte_f(wq, t) - 8.0f;
                            a = fmaf(dd * q, xs[t], a);  // fl(d*q) is exact for these codes
                        }
                    }
                }
            }
            }
            }
            v[s] = active ? a : 0.0f;
            if (i0 + s + PD < RPW) load_row(R[slot], row_of(i0 + s + PD));  // refill the slot just consumed
        }
        float sum = lane_sum8(v, lane);
        const int ri = lane >> 3;
        if (KS > 1) {
            float *pl = part_lds[(i0 >> 3) & 1];
            if (part && (lane & 7) == 0) pl[((part - 1) * RG + rg) * 8 + ri] = sum;
            __syncthreads();
            if (!part) {
#pragma unroll
                for (int q = 1; q < KS; q++) sum = sum + pl[((q - 1) * RG + rg) * 8 + ri];
            }
        }
        if constexpr (SWI) {  // rows ri (even: gate) and ri + 1 (up) of the eight are lanes 8 ri and 8 ri + 8
            const float up = __shfl_xor(sum, 8);
            const uint32_t j = (uint32_t)(i0 + ri) >> 1;
            if (part == 0 && (lane & 15) == 0 && j < nv) c[gw + (int64_t)j * G] = silu_ref(sum) * up;
        } else {
            const int64_t r = gw + (int64_t)(i0 + ri) * G;
            if (part == 0 && (lane & 7) == 0 && (uint32_t)(i0 + ri) < nv) {
                if constexpr (IO == TRHIP_F32) {
                    c[r] = ACC ? c[r] + sum : sum;
                } else {  // c widened, the sum added in fp32, rounded once
                    uint16_t *c16 = static_cast<uint16_t *>(cv);
                    c16[r] = (uint16_t)f32_to_h16(ACC ? h16_to_f32(c16[r], IO) + sum : sum, IO);
                }
            }
        }
    }
}

// Whether the K-across-lanes kernel takes a store with nb blocks per row in KS parts: q4_k / q6_k parts of at
// most 16 blocks; q8_0 / q4_0 an even block count and parts of at most 128 blocks (two per lane).
__host__ __forceinline__ bool kl_fits(int dt, int64_t nb, int ks) {
    if (dt == kQ4K || dt == kQ6K) return (nb + ks - 1) / ks <= 16;
    return nb % 2 == 0 && ((nb + ks - 1) / ks + 1) / 2 * 2 <= 128;
}

template <int DT, int WAVES, int KS, int PD, int RPW, bool SWI = false, int IO = TRHIP_F32>
int run_kl(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c, bool acc) {
    constexpr int RG = WAVES / KS;
    if (!kl_fits(DT, w->nb, KS)) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemv_kl: K parts too long for the lanes of a wave");
    constexpr int OPW = SWI ? RPW / 2 : RPW;  // outputs per row group (SWI: two rows per output)
    int64_t wgs = (N + RG * OPW - 1) / (RG * OPW);  // every row group gets at most RPW rows
    // Fewer workgroups than CUs: deal the rows over one workgroup per CU (at least one output per row group, the
    // shorter groups skipping their spare slots). Cold ring, us (same box, interleaved): q6_k 1024x4096 7.70 ->
    // 5.73, q4_0 4096x4096 5.45 -> 4.68, q6_k 4096x4096 8.02 -> 7.38, q4_k 6144x4096 5.56 -> 5.37 (with SwiGLU
    // 5.63 -> 5.46); at 14336 rows (16 -> 14 rows per group) q4_k 8.03 -> 7.74-7.85, q8_0 12.86 -> 12.55, q6_k
    // 11.96 -> 11.83, but q4_0 7.64 -> 7.89, so q4_0 spreads only where a group keeps at most 3/4 of its rows.
    const int64_t cus = ctx->sm_count > 0 ? ctx->sm_count : 256, cap = (N + RG - 1) / RG;
    const int64_t spread = cus < cap ? cus : cap, per = (N + spread * RG - 1) / (spread * RG);
    int64_t wide = wgs < cus && (DT != kQ4 || 4 * per <= 3 * OPW) ? spread : wgs;
    if (ctx->kl_min_wgs > wide) wide = ctx->kl_min_wgs;  // more, shorter row groups (forced for tuning)
    const bool skip = wide > wgs;
    wgs = wide;
    if (N >= (int64_t)1 << 30 || wgs * RG >= (int64_t)1 << 31)
        return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemv_kl: more than 2^30 rows");
    dim3 grid((unsigned)wgs), block(64 * WAVES);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, ctx->stream, w->planes(), x, c, N, row0);
        return launch_check(ctx, SWI ? "gemv_kl_swiglu" : "gemv_kl");
    };
    if constexpr (SWI)
        return skip ? go(gemv_kl<DT, false, WAVES, KS, PD, RPW, true, true>)
                    : go(gemv_kl<DT, false, WAVES, KS, PD, RPW, true, false>);
    if (acc)
        return skip ? go(gemv_kl<DT, true, WAVES, KS, PD, RPW, false, true, IO>)
                    : go(gemv_kl<DT, true, WAVES, KS, PD, RPW, false, false, IO>);
    return skip ? go(gemv_kl<DT, false, WAVES, KS, PD, RPW, false, true, IO>)
                : go(gemv_kl<DT, false, WAVES, KS, PD, RPW, false, false, IO>);
}

template <int D, int WAVES, int KS, int R>
int run_q4k(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc) {
    constexpr int ROWS = 8 * R * WAVES / KS;
    const int64_t nx4 = w->K / 4;
    size_t lds = (size_t)(nx4 + nx4 / 16) * sizeof(float4) + (size_t)(w->K / 16) * sizeof(float);
    if (lds > 150 * 1024) return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemv_fast: K too large for the LDS copy of x");
    dim3 grid((unsigned)((N + ROWS - 1) / ROWS)), block(64 * WAVES);
    if (lds > 62 * 1024) {  // with the kernel's static LDS above 64 KB (K > ~13800): allowed once per device
        int st = allow_dyn_lds(ctx, reinterpret_cast<const void *>(&gemv_fast_q4k<true, D, WAVES, KS, R>), lds,
                               "gemv_fast_q4k: LDS size");
        if (st == TRHIP_OK)
            st = allow_dyn_lds(ctx, reinterpret_cast<const void *>(&gemv_fast_q4k<false, D, WAVES, KS, R>), lds,
                               "gemv_fast_q4k: LDS size");
        if (st != TRHIP_OK) return st;
    }
    if (acc)
        hipLaunchKernelGGL((gemv_fast_q4k<true, D, WAVES, KS, R>), grid, block, lds, ctx->stream, w->planes(), x, c, N, row0, w->K);
    else
        hipLaunchKernelGGL((gemv_fast_q4k<false, D, WAVES, KS, R>), grid, block, lds, ctx->stream, w->planes(), x, c, N, row0, w->K);
    return launch_check(ctx, "gemv_fast_q4k");
}

}  // namespace

int launch_gemv(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc,
                int mode);

namespace {
// K across lanes with the launch shape forced on the context (trhip_set_launch_shape, tests and tuning), or
// kNotTaken when none is.
constexpr int kNotTaken = -1;
template <int DT>
int kl_forced(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc) {
    switch (ctx->force_kl) {
    case 0: return kNotTaken;
    case 4141: return run_kl<DT, 4, 1, 4, 8>(ctx, w, row0, N, x, c, acc);
    case 4142: return run_kl<DT, 4, 1, 4, 16>(ctx, w, row0, N, x, c, acc);
    case 4122: return run_kl<DT, 4, 1, 2, 16>(ctx, w, row0, N, x, c, acc);
    case 8141: return run_kl<DT, 8, 1, 4, 8>(ctx, w, row0, N, x, c, acc);
    case 4242: return run_kl<DT, 4, 2, 4, 16>(ctx, w, row0, N, x, c, acc);
    case 4241: return run_kl<DT, 4, 2, 4, 8>(ctx, w, row0, N, x, c, acc);
    case 8241: return run_kl<DT, 8, 2, 4, 8>(ctx, w, row0, N, x, c, acc);
    case 8441: return run_kl<DT, 8, 4, 4, 8>(ctx, w, row0, N, x, c, acc);
    case 4181: return run_kl<DT, 4, 1, 8, 8>(ctx, w, row0, N, x, c, acc);
    case 8181: return run_kl<DT, 8, 1, 8, 8>(ctx, w, row0, N, x, c, acc);
    case 2181: return run_kl<DT, 2, 1, 8, 8>(ctx, w, row0, N, x, c, acc);
    case 4182: return run_kl<DT, 4, 1, 8, 16>(ctx, w, row0, N, x, c, acc);
    case 16181: return run_kl<DT, 16, 1, 8, 8>(ctx, w, row0, N, x, c, acc);
    case 4441: return run_kl<DT, 4, 4, 4, 8>(ctx, w, row0, N, x, c, acc);
    case 8442: return run_kl<DT, 8, 4, 4, 16>(ctx, w, row0, N, x, c, acc);
    }
    return fail(ctx, TRHIP_ERR_UNSUPPORTED, "gemv_kl: no such launch shape");
}

// q8_0 / q4_0: K across lanes where the store fits it, else the exact kernel (within any tolerance)
template <int DT>
int kl_q8q4(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc) {
    const int f = kl_forced<DT>(ctx, w, row0, N, x, c, acc);
    if (f != kNotTaken) return f;
    // cold 1.1 GiB rings (us): q8_0 4096 x 4096 6.21-6.23 in one K part, 6.38-6.41 in two (with the row arithmetic
    // of the current kernel; two parts were faster before it, 6.9 against 7.2), 14336 x 4096 12.5 with 16 rows per
    // wave; q4_0 4096 x 4096 5.5 / 6.2, 14336 x 4096 8.2; K = 14336 takes four parts (q8_0 15.0, q4_0 10.7)
    if (kl_fits(DT, w->nb, 1)) {
        if (N >= 10240) return run_kl<DT, 4, 1, 4, 16>(ctx, w, row0, N, x, c, acc);
        return run_kl<DT, 4, 1, 4, 8>(ctx, w, row0, N, x, c, acc);
    }
    if (kl_fits(DT, w->nb, 4)) return run_kl<DT, 8, 4, 4, 8>(ctx, w, row0, N, x, c, acc);
    return kNotTaken;
}

// q6_k: K across lanes (K up to 4096 in one part, K up to 16384 in four), else the exact kernel
int kl_q6k(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c, bool acc) {
    const int f = kl_forced<kQ6K>(ctx, w, row0, N, x, c, acc);
    if (f != kNotTaken) return f;
    if (kl_fits(kQ6K, w->nb, 1)) {
        if (N >= 10240) return run_kl<kQ6K, 4, 1, 4, 16>(ctx, w, row0, N, x, c, acc);
        return run_kl<kQ6K, 4, 1, 4, 8>(ctx, w, row0, N, x, c, acc);
    }
    if (kl_fits(kQ6K, w->nb, 4)) return run_kl<kQ6K, 8, 4, 4, 8>(ctx, w, row0, N, x, c, acc);
    return kNotTaken;
}
}  // namespace

// q4_k GEMV with the SwiGLU gate fused (merged [gate | up] store of 2I rows, M = 1): the K-across-lanes launch
// shape the unfused fast GEMV takes for 2I rows, so every row sum, and so every gated output, has the same bits
int launch_gemv_fast_swiglu(trhip_ctx *ctx, const trhip_wstore *w, const float *x, float *out, int64_t I) {
    const int64_t N2 = 2 * I;
    if (w->dtype != kQ4K || w->N != N2 || ctx->force_kl || w->nb < 8 || w->nb > 16) return kNotTaken;
    if (N2 >= 10240) return run_kl<kQ4K, 4, 1, 4, 16, true>(ctx, w, 0, I, x, out, false);
    if (N2 >= 6144) return run_kl<kQ4K, 4, 1, 4, 8, true>(ctx, w, 0, I, x, out, false);
    return kNotTaken;
}

int launch_gemv_fast(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     bool acc) {
    if (w->dtype == kQ6K) {
        const int r = kl_q6k(ctx, w, row0, N, x, c, acc);
        if (r != kNotTaken) return r;
    }
    if (w->dtype == kQ8 || w->dtype == kQ4) {
        const int r = w->dtype == kQ8 ? kl_q8q4<kQ8>(ctx, w, row0, N, x, c, acc) : kl_q8q4<kQ4>(ctx, w, row0, N, x, c, acc);
        if (r != kNotTaken) return r;
    }
    if (w->dtype == kQ4K) {
        const int f = kl_forced<kQ4K>(ctx, w, row0, N, x, c, acc);
        if (f != kNotTaken) return f;
        // Measured on cold 1.1 GiB rings (us), K = 4096: 14336 rows 8.6 K across lanes (16 rows per wave) vs
        // 11.6-12.2 row-sliced, 28672 rows 14.7 vs 15.9 with 8 rows per wave; 6144 / 8192 rows 5.6 / 5.8 with 8 rows
        // per wave vs 7.9 / 8.0 with 16 and 6.2-6.5 / 8.0 row-sliced; with the rows of small grids spread over every
        // CU (run_kl), 4096 / 1024 rows 4.79 / 3.95 vs 4.95 / 4.20 row-sliced. Below 8 blocks per row lanes would
        // idle.
        // trhip_set_launch_shape(TRHIP_KNOB_FAST_Q4K) selects the row-sliced kernel.
        const bool kl_ok = !ctx->force_fast_q4k && w->nb >= 8 && w->nb <= 16;
        if (kl_ok && N >= 10240) return run_kl<kQ4K, 4, 1, 4, 16>(ctx, w, row0, N, x, c, acc);
        if (kl_ok) return run_kl<kQ4K, 4, 1, 4, 8>(ctx, w, row0, N, x, c, acc);
        // K of 17..64 blocks from 4096 rows: four K parts (4096x14336, cold: 10.25-10.33 us against 10.48-10.66
        // row-sliced)
        if (!ctx->force_fast_q4k && w->nb > 16 && kl_fits(kQ4K, w->nb, 4) && N >= 4096)
            return run_kl<kQ4K, 8, 4, 4, 8>(ctx, w, row0, N, x, c, acc);
        // launch shape "D,WAVES,KS,R": blocks in flight per lane, waves per workgroup, K parts per row group,
        // rows per lane. Measured on cold 1.1 GiB rings: splitting K wins while the grid is small (1024 / 4096 rows
        // at K = 4096: 5.5 / 5.9 us with 2 parts vs 7.9 / 8.2 whole), whole rows per wave win from ~8192 rows
        // (14336 rows: 10.7-11.5 us vs 11.6-11.7). More blocks in flight or more rows per lane were slower.
        const int forced = ctx->force_fast_q4k;
        // K split in 4 for fewer rows (cold, us): 4096x14336 10.9 vs 14.5 (2 parts), 4096x4096 5.1 vs 6.0,
        // 1024x14336 8.3 vs 12.8
        const int cfg = forced ? forced : (N >= 8192 ? 2411 : (N >= 2048 ? 2841 : 2441));
        switch (cfg) {
        case 2441: return run_q4k<2, 4, 4, 1>(ctx, w, row0, N, x, c, acc);
        case 2841: return run_q4k<2, 8, 4, 1>(ctx, w, row0, N, x, c, acc);
        case 2421: return run_q4k<2, 4, 2, 1>(ctx, w, row0, N, x, c, acc);
        case 2411: return run_q4k<2, 4, 1, 1>(ctx, w, row0, N, x, c, acc);
        case 2422: return run_q4k<2, 4, 2, 2>(ctx, w, row0, N, x, c, acc);
        case 8421: return run_q4k<8, 4, 2, 1>(ctx, w, row0, N, x, c, acc);
        }
        return run_q4k<2, 4, 2, 1>(ctx, w, row0, N, x, c, acc);
    }
    return launch_gemv(ctx, w, row0, N, x, c, acc, TRHIP_MODE_EXACT);
}

// 16-bit x and c on the K-across-lanes kernel: the same launch shapes launch_gemv_fast takes for each dtype and store
// shape (so the row sums are those of the fp32 call on the widened x), kNotTaken where it would take another kernel
// or a launch shape is forced on the context.
namespace {
template <int IO>
int gemv_fast_io(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c, bool acc) {
    if (ctx->force_kl || ctx->force_fast_q4k || ctx->kl_min_wgs) return kNotTaken;
    switch (w->dtype) {
    case kQ4K:
        if (w->nb >= 8 && w->nb <= 16)
            return N >= 10240 ? run_kl<kQ4K, 4, 1, 4, 16, false, IO>(ctx, w, row0, N, x, c, acc)
                              : run_kl<kQ4K, 4, 1, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc);
        if (w->nb > 16 && kl_fits(kQ4K, w->nb, 4) && N >= 4096)
            return run_kl<kQ4K, 8, 4, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc);
        return kNotTaken;
    case kQ6K:
        if (kl_fits(kQ6K, w->nb, 1))
            return N >= 10240 ? run_kl<kQ6K, 4, 1, 4, 16, false, IO>(ctx, w, row0, N, x, c, acc)
                              : run_kl<kQ6K, 4, 1, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc);
        if (kl_fits(kQ6K, w->nb, 4)) return run_kl<kQ6K, 8, 4, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc);
        return kNotTaken;
    case kQ8:
    case kQ4:
        if (kl_fits(w->dtype, w->nb, 1)) {
            if (w->dtype == kQ8)
                return N >= 10240 ? run_kl<kQ8, 4, 1, 4, 16, false, IO>(ctx, w, row0, N, x, c, acc)
                                  : run_kl<kQ8, 4, 1, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc);
            return N >= 10240 ? run_kl<kQ4, 4, 1, 4, 16, false, IO>(ctx, w, row0, N, x, c, acc)
                              : run_kl<kQ4, 4, 1, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc);
        }
        if (kl_fits(w->dtype, w->nb, 4))
            return w->dtype == kQ8 ? run_kl<kQ8, 8, 4, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc)
                                   : run_kl<kQ4, 8, 4, 4, 8, false, IO>(ctx, w, row0, N, x, c, acc);
        return kNotTaken;
    }
    return kNotTaken;
}
}  // namespace

int launch_gemv_fast_io(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                        bool acc, int io) {
    if (N == 0) return TRHIP_OK;
    if (io == TRHIP_F16) return gemv_fast_io<TRHIP_F16>(ctx, w, row0, N, x, c, acc);
    if (io == TRHIP_BF16) return gemv_fast_io<TRHIP_BF16>(ctx, w, row0, N, x, c, acc);
    return kNotTaken;
}

}  // namespace trhip
