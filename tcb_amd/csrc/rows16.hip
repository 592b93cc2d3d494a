// rows16.hip -- fast-mode (tolerance) q4_k and q4_0 product for 1..16 activation rows in one launch: the batched
// decode step (c[m, n] (+)= sum_k x[m, k] w[n, k], the reference's quantGemm at small M, tensor/cpu_quant.go:47-147;
// its GPU twin runs M > 1 as dequantized tiles through a float GEMM, gpu/backend_quant.go:43-134).
// q4_0 (y = d (q - 8) per 32-element block, tensor/quant.go:149-155) takes the same staging and activation record
// with one MFMA pair per block: D_b = sum (q - 8)(hi + lo) in fp32, acc += d_b D_b.
//
// Arithmetic, per 256-element block b of activation row m (2^E > the block's largest |x|):
//   x' = x 2^(11-E), held as two f16 terms hi = f16(x'), lo = f16(x' - hi): hi + lo is x' to about 2^-22 of 2^11.
//   The weights enter the f16 MFMA as the exact products q sc (q < 16, sc < 64: q sc <= 945 is an f16 integer),
//   made from the nibbles by one bit operation per two codes, 0x6400 | nibble (the f16 1024 + q, or 1024 + 16 q
//   for a high nibble left in place), and one packed f16 fma: (1024 + q) sc - 1024 sc, (1024 + 16 q) (sc/16) - 64 sc,
//   exact because the fma rounds once and the result is a small integer.
//   One fp32 accumulator therefore takes the whole block, D = sum (q sc) (hi + lo); the minimum term
//   Mn = sum_j m_j sum_{k in j} x'_k is one 16x16x16 f16 MFMA over the 32-element sums (two f16 terms each, scaled
//   by 1/32 so they stay in range, with 32 m_j as the other operand); per block and output
//   acc += ldexp(d D - dmin Mn, E - 11).
// Rows of x holding NaN / Inf take exact float dot products (slice by slice), as in the other fast kernels.
//
// Grid: a workgroup is 4 waves over R = 64 TPW weight rows (wave w: TPW tiles of 16 rows; lane l of a tile owns row
// l % 16 and qs pair g = l / 16, i.e. sub-blocks 2g, 2g + 1) and a K slice of bps blocks. Per block the workgroup
// turns the 16 x 256 activations into the f16 operands in LDS (double-buffered, one barrier per block) while its
// weights for the next block are in flight. With one slice the results go straight to c; with S > 1 each
// workgroup writes its slice's partial tile, and the workgroup that arrives last at the row tile's counter adds the
// S partials in slice order (fixed, so the result does not depend on arrival order) and writes c, then returns the
// counter to zero. The SwiGLU variant gives a workgroup gate rows i0 .. i0 + R/2 and up rows I + i0 .. so the last
// workgroup holds both halves of its outputs: out = silu(g) u, with g and u summed as the plain kernel sums them.
#include "trhip_internal.hpp"
#include "mfma_util.hpp"

#include <cfloat>

namespace trhip {
namespace {

constexpr int R16_THREADS = 256;
constexpr int R16_PLANE = 8 * 64 * 16;  // one f16 plane of a block: step s x lane x 8 halves
// activation record of a block: hi plane, lo plane, msum operands (lane x 4 halves), exponents and NaN / Inf flags
// of the 16 rows, padding to 1 KB after the planes
constexpr int R16_XSO = 2 * R16_PLANE, R16_EXO = R16_XSO + 512, R16_BADO = R16_EXO + 64;
constexpr int R16_XREC = 2 * R16_PLANE + 1024;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct R16W {  // one tile's registers for one block: the lane's 32 qs bytes (pair g) and the block header
    u32x4 a, b, h;
};

// Repacked q4_k qs: bytes [16g, 16g + 16) hold original bytes 32g .. 32g + 15 and [64 + 16g, +16) bytes
// 32g + 16 .. 32g + 31 (trhip_internal.hpp), so the lane's pair is two 16-byte loads.
__device__ __forceinline__ void r16_load(R16W &r, const Planes p, int64_t row, int64_t blk, int g) {
    const int64_t bi = row * p.nb + blk;
    r.a = *reinterpret_cast<const u32x4 *>(p.qs + bi * 128 + 16 * g);
    r.b = *reinterpret_cast<const u32x4 *>(p.qs + bi * 128 + 64 + 16 * g);
    r.h = *reinterpret_cast<const u32x4 *>(p.aux + bi * 16);
}

struct R16K {  // per tile and block: f16 multipliers / offsets of the lane's two sub-blocks, msum operand, d, dmin
    h2 mul, off;  // (sc_2g, sc_2g+1 / 16), (-1024 sc_2g, -64 sc_2g+1)
    v4h mB;       // 32 (m_2g, m_2g, m_2g+1, m_2g+1)
    float d, dmin;
};

__device__ __forceinline__ h2 f16_bytes(uint32_t w, uint32_t sel) {  // two bytes of w as f16 1024 + byte
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w, sel));
}

__device__ __forceinline__ void r16_consts(R16K &k, const R16W &r, int g) {
    uint32_t sc_lo, sc_hi, m_lo, m_hi;
    q4k_scales(r.h.y, r.h.z, r.h.w, sc_lo, sc_hi, m_lo, m_hi);  // tensor/quant.go:158-163
    const uint32_t scw = g < 2 ? sc_lo : sc_hi, mw = g < 2 ? m_lo : m_hi;
    const uint32_t sel = (g & 1) ? 0x04030402u : 0x04010400u;  // bytes 2g, 2g + 1 of the four
    const h2 base = (h2){(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 sp = f16_bytes(scw, sel) - base, mp = f16_bytes(mw, sel) - base;
    k.mul = sp * (h2){(_Float16)1.0f, (_Float16)0.0625f};
    k.off = sp * (h2){(_Float16)-1024.0f, (_Float16)-64.0f};
    const _Float16 m32 = (_Float16)32.0f;
    k.mB = (v4h){mp.x * m32, mp.x * m32, mp.y * m32, mp.y * m32};
    k.d = f16_to_f32((uint16_t)(r.h.x & 0xFFFFu));
    k.dmin = f16_to_f32((uint16_t)(r.h.x >> 16));
}

// The 8 operand halves of step s (qs dword s of the pair: bytes 32g + 4s .. + 3) as exact q sc, in the order
// (byte 0, 2, 1, 3) low nibbles, then the same bytes' high nibbles; the activation planes use the same order.
// (k6464 = 0x64006400 in a register: with the mask as the one literal, each pair is one v_and_or_b32)
__device__ __forceinline__ v8h r16_codes(const R16W &r, const R16K &k, int s, uint32_t k6464) {
    const uint32_t wd = s == 0 ? r.a.x : s == 1 ? r.a.y : s == 2 ? r.a.z : s == 3 ? r.a.w
                      : s == 4 ? r.b.x : s == 5 ? r.b.y : s == 6 ? r.b.z : r.b.w;
    const uint32_t w8 = wd >> 8;
    const h2 p0 = __builtin_bit_cast(h2, (wd & 0x000F000Fu) | k6464);
    const h2 p1 = __builtin_bit_cast(h2, (wd & 0x00F000F0u) | k6464);
    const h2 p2 = __builtin_bit_cast(h2, (w8 & 0x000F000Fu) | k6464);
    const h2 p3 = __builtin_bit_cast(h2, (w8 & 0x00F000F0u) | k6464);
    const h2 ml = (h2){k.mul.x, k.mul.x}, ol = (h2){k.off.x, k.off.x};
    const h2 mh = (h2){k.mul.y, k.mul.y}, oh = (h2){k.off.y, k.off.y};
    const h2 q0 = __builtin_elementwise_fma(p0, ml, ol), q2 = __builtin_elementwise_fma(p2, ml, ol);
    const h2 q1 = __builtin_elementwise_fma(p1, mh, oh), q3 = __builtin_elementwise_fma(p3, mh, oh);
    return (v8h){q0.x, q0.y, q2.x, q2.y, q1.x, q1.y, q3.x, q3.y};
}

// One WG per 256-element block: the 16 x 256 activations as the f16 operand record of the block (hi plane, lo
// plane, msum operands, exponents, NaN / Inf flags), laid out as the MFMA reads them (step s, lane l at 64 s + l).
// q4_0 (DT = kQ4): step s is 32-element block s of the 256, and lane group gq holds its elements 4 gq + (0, 2, 1, 3)
// (the low nibbles of code bytes 4 gq .. 4 gq + 3) and 16 + 4 gq + (0, 2, 1, 3) (their high nibbles); no msum.
// IO: fp32 x, or f16 / bf16 x widened exactly on load (the record is then that of the widened x).
template <int DT, int IO = TRHIP_F32>
__global__ __launch_bounds__(R16_THREADS) void halves16_kernel(const void *__restrict__ xv, int64_t M, int64_t K,
                                                               uint8_t *__restrict__ rec) {
    const int b = blockIdx.x, tid = threadIdx.x;
    uint8_t *st = rec + (int64_t)b * R16_XREC;
    // thread (pm, pu) holds elements 16 pu .. 16 pu + 15 of row pm of the block
    const int pm = tid >> 4, pu = tid & 15;
    const bool prow = pm < M;
    const int64_t e0 = (prow ? pm : 0) * K + 256 * (int64_t)b + 16 * pu;
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 q;
        if constexpr (IO == TRHIP_F32) {
            q = reinterpret_cast<const float4 *>(static_cast<const float *>(xv) + e0)[i];
        } else {
            const uint2 hh = reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(xv) + e0)[i];
            q = make_float4(h16_to_f32(hh.x & 0xFFFFu, IO), h16_to_f32(hh.x >> 16, IO), h16_to_f32(hh.y & 0xFFFFu, IO),
                            h16_to_f32(hh.y >> 16, IO));
        }
        v[4 * i] = prow ? q.x : 0.0f;
        v[4 * i + 1] = prow ? q.y : 0.0f;
        v[4 * i + 2] = prow ? q.z : 0.0f;
        v[4 * i + 3] = prow ? q.w : 0.0f;
    }
    float amax = 0.0f;
    bool fin = true;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        amax = fmaxf(amax, fabsf(v[j]));
        fin = fin && fabsf(v[j]) <= FLT_MAX;
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const uint64_t badm = __ballot(!fin);
    const bool bad = ((badm >> (16 * ((tid >> 4) & 3))) & 0xFFFFull) != 0;
    int E = 0;
    if (!bad && amax > 0.0f) frexpf(amax, &E);  // amax = f 2^E, f in [0.5, 1)
    float xs[16];
#pragma unroll
    for (int j = 0; j < 16; j++) xs[j] = bad ? 0.0f : ldexpf(v[j], 11 - E);  // |xs| < 2^11
    // element 16 pu + j is sub-block 2 gq + half, element i = 16 (pu & 1) + j of it: step i / 4, operand half
    // `half`, position (0, 2, 1, 3)[i % 4] (the weight operand's code order)
    const int gq = pu >> 2, half = (pu >> 1) & 1, s0 = 4 * (pu & 1);
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const float a[4] = {xs[4 * jj], xs[4 * jj + 2], xs[4 * jj + 1], xs[4 * jj + 3]};
        uint16_t hb[4], lb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const _Float16 h = (_Float16)a[i];
            hb[i] = __builtin_bit_cast(uint16_t, h);
            lb[i] = __builtin_bit_cast(uint16_t, (_Float16)(a[i] - (float)h));
        }
        // q4_0: this thread's 16 elements are half pu & 1 of block pu >> 1, elements 4 jj .. 4 jj + 3 of it lane group jj
        const int slot = DT == kQ4 ? (64 * (pu >> 1) + 16 * jj + pm) * 16 + 8 * (pu & 1)
                                   : (64 * (s0 + jj) + 16 * gq + pm) * 16 + 8 * half;
        *reinterpret_cast<uint2 *>(st + slot) =
            make_uint2(hb[0] | ((uint32_t)hb[1] << 16), hb[2] | ((uint32_t)hb[3] << 16));
        *reinterpret_cast<uint2 *>(st + R16_PLANE + slot) =
            make_uint2(lb[0] | ((uint32_t)lb[1] << 16), lb[2] | ((uint32_t)lb[3] << 16));
    }
    const float sum = (((xs[0] + xs[1]) + (xs[2] + xs[3])) + ((xs[4] + xs[5]) + (xs[6] + xs[7]))) +
                      (((xs[8] + xs[9]) + (xs[10] + xs[11])) + ((xs[12] + xs[13]) + (xs[14] + xs[15])));
    const float xsum = (sum + __shfl_xor(sum, 1)) * 0.03125f;  // the 32-element sum / 32: |.| < 2^11
    if (DT == kQ4K && (pu & 1) == 0) {  // msum A operand: lane (m, kq) holds (hi, lo) of sub-blocks 2 kq, 2 kq + 1
        const _Float16 h = (_Float16)xsum;
        const uint32_t pr = (uint32_t)__builtin_bit_cast(uint16_t, h) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(xsum - (float)h)) << 16);
        *reinterpret_cast<uint32_t *>(st + R16_XSO + (16 * gq + pm) * 8 + 4 * half) = pr;
    }
    if (pu == 0) {
        reinterpret_cast<int *>(st + R16_EXO)[pm] = E - 11;
        reinterpret_cast<int *>(st + R16_BADO)[pm] = bad ? 1 : 0;
    }
}

typedef __attribute__((address_space(3))) void *lds_ptr;
// Raw buffer over [base, base + bytes): 32-bit offsets per lane; reads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t r16_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// SIZE bytes per lane from rsrc at voffset + soffset into LDS at l + SIZE * lane (l wave-uniform). (A device
// function: written inline in the kernel, the cast of a static LDS array's address keeps the host pass from
// emitting the kernel's launch stub.)
__device__ __forceinline__ void r16_dma16(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset, void *l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)l, 16, voffset, soffset, 0, 0);
}
__device__ __forceinline__ void r16_dma4(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset, void *l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)l, 4, voffset, soffset, 0, 0);
}
#define R16_DMA(SIZE, r, voffset, soffset, l) r16_dma##SIZE((r), (voffset), (soffset), (l))

// s_waitcnt vmcnt(n) leaving the other counters alone (gfx9 encoding: vmcnt [3:0] and [15:14], expcnt [6:4],
// lgkmcnt [11:8])
#define R16_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

template <int TPW>
struct R16Stage {  // one block in LDS: the activation record, the R rows' headers, their qs (16-byte pieces swizzled)
    static constexpr int R = 64 * TPW;
    static constexpr int HDR = R16_XREC;
    static constexpr int QS = HDR + 16 * R;
    static constexpr int BYTES = QS + 128 * R;
    static constexpr int DMAS = 5 + 3 * TPW;  // DMA instructions per thread and stage
};

// DT: q4_k, or q4_0 (its 256-element chunk holds eight blocks: the 16-byte header of a row's chunk is the blocks'
// eight fp16 scales, its 128 qs bytes their codes, so the staging is the same)
// (two waves per SIMD, which the LDS allows anyway: with the register budget of that occupancy the products stay in
// VGPRs rather than being copied out of the accumulator registers)
// IO: fp32 x and c, or f16 / bf16 x and c (x widened exactly, c widened, the fp32 result added, rounded once);
// not with SWI, whose gated output is fp32
template <int DT, int TPW, bool ACC, bool SWI, int IO = TRHIP_F32>
__global__ __launch_bounds__(R16_THREADS) __attribute__((amdgpu_waves_per_eu(2, 2))) void rows16_gemm(const Planes p, int64_t nrows, int64_t N, int64_t row0,
                                                           int64_t M, int64_t K, const void *__restrict__ xv,
                                                           const uint8_t *__restrict__ rec, int64_t RT, int S, int bps,
                                                           void *__restrict__ cv, float *__restrict__ part,
                                                           uint32_t *__restrict__ arrivals) {
    static_assert(DT == kQ4K || (DT == kQ4 && !SWI), "q4_k, or q4_0 without the gate");
    static_assert(IO == TRHIP_F32 || !SWI, "the gated output is fp32");
    float *c = static_cast<float *>(cv);  // (IO == TRHIP_F32)
    auto xat = [&](int64_t i) -> float {  // element i of x, widened
        if constexpr (IO == TRHIP_F32) return static_cast<const float *>(xv)[i];
        else return h16_to_f32(static_cast<const uint16_t *>(xv)[i], IO);
    };
    auto cput = [&](int64_t i, float v) {  // c[i] (+)= v, rounded once when 16-bit
        if constexpr (IO == TRHIP_F32) {
            c[i] = ACC ? c[i] + v : v;
        } else {
            uint16_t *c16 = static_cast<uint16_t *>(cv);
            c16[i] = (uint16_t)f32_to_h16(ACC ? h16_to_f32(c16[i], IO) + v : v, IO);
        }
    };
    using T = R16Stage<TPW>;
    constexpr int R = T::R, H = R / 2;
    // three stages as separate arrays: the compiler then sees that the reads of one stage do not alias the DMA
    // into another, and does not wait for the later blocks' loads before computing the current one
    __shared__ __align__(16) uint8_t st0[T::BYTES];
    __shared__ __align__(16) uint8_t st1[T::BYTES];
    __shared__ __align__(16) uint8_t st2[T::BYTES];
    __shared__ int rowbad[16];
    __shared__ int lastflag;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = (int)(K / 256);
    // workgroup -> (row tile, slice): workgroups are dealt to the 8 XCDs in turn, so consecutive indices t in one
    // XCD take the row tiles of one slice, whose activation records then stay in that XCD's L2
    const int64_t total = RT * S;
    int64_t t = blockIdx.x;
    if (total % 8 == 0) t = (int64_t)(blockIdx.x & 7) * (total / 8) + (blockIdx.x >> 3);
    const int sl = (int)(t / RT);
    const int64_t rt = t - (int64_t)sl * RT;
    const int c0 = sl * bps, c1 = c0 + bps < nb ? c0 + bps : nb;
    const int64_t I = N / 2;
    auto out_row = [&](int nl) -> int64_t {  // store row of local row nl (before row0)
        if (SWI) return nl < H ? rt * H + nl : I + rt * H + (nl - H);
        return rt * R + nl;
    };
    auto row_ok = [&](int nl) -> bool {
        if (SWI) return rt * H + (nl < H ? nl : nl - H) < I;
        return rt * R + nl < N;
    };
    auto srow = [&](int nl) -> int64_t { return row0 + (row_ok(nl) ? out_row(nl) : 0); };

    // DMA offsets of this thread (the block adds a wave-uniform offset): qs piece P = 256 i + tid is local row
    // P / 8, piece (P % 8) ^ (row % 8), so that the reads of 16 rows' same piece fall in different banks; header
    // dword 256 i + tid is row / 4, word % 4; the activation record is copied as it is
    const auto rx = r16_rsrc(rec, (uint32_t)(nb * R16_XREC));
    const auto rq = r16_rsrc(p.qs, (uint32_t)(nrows * nb * 128));
    const auto rh = r16_rsrc(DT == kQ4 ? static_cast<const void *>(p.d) : static_cast<const void *>(p.aux),
                             (uint32_t)(nrows * nb * 16));
    uint32_t vq[2 * TPW], vh[TPW];
#pragma unroll
    for (int i = 0; i < 2 * TPW; i++) {
        const int P = 256 * i + tid, r = P >> 3, q = P & 7;
        vq[i] = (uint32_t)(srow(r) * nb * 128 + 16 * (q ^ (r & 7)));
    }
#pragma unroll
    for (int i = 0; i < TPW; i++) {
        const int D = 256 * i + tid, r = D >> 2;
        vh[i] = (uint32_t)(srow(r) * nb * 16 + 4 * (D & 3));
    }
    auto stage = [&](uint8_t *sb, int b) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            R16_DMA(16, rx, (uint32_t)(16 * (256 * i + tid)), (uint32_t)(b * R16_XREC), sb + 4096 * i + 1024 * w);
        R16_DMA(4, rx, (uint32_t)(2 * R16_PLANE + 4 * tid), (uint32_t)(b * R16_XREC), sb + 2 * R16_PLANE + 256 * w);
#pragma unroll
        for (int i = 0; i < TPW; i++) R16_DMA(4, rh, vh[i], (uint32_t)(16 * b), sb + T::HDR + 1024 * i + 256 * w);
#pragma unroll
        for (int i = 0; i < 2 * TPW; i++) R16_DMA(16, rq, vq[i], (uint32_t)(128 * b), sb + T::QS + 4096 * i + 1024 * w);
    };

    float acc[TPW][4];
#pragma unroll
    for (int tt = 0; tt < TPW; tt++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[tt][r] = 0.0f;
    int badrow = 0;
    auto last = [&](int b) { return b < c1 ? b : c1 - 1; };

    const uint32_t k6464 = opaque(0x64006400u);  // in a register, so the nibble masks fuse into v_and_or_b32
    const v4f zero = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    auto compute_q4 = [&](const uint8_t *cur) {
        // q4_0: lane (n, g) of a tile takes code dword g of each block s (low nibbles: elements 4g + (0, 2, 1, 3),
        // high: 16 + 4g + ...), as exact f16 q - 8 ((1024 + q) - 1032, (1024 + 16 q) / 16 - 72); per block the two
        // MFMAs give D_s = sum (q - 8)(hi + lo) for the tile, scaled by the row's d_s; per chunk acc += ldexp(., E - 11)
        R16W cw[TPW];
        R16K k;
        k.mul = (h2){(_Float16)1.0f, (_Float16)0.0625f};
        k.off = (h2){(_Float16)-1032.0f, (_Float16)-72.0f};
        float ds[TPW][8];
#pragma unroll
        for (int tt = 0; tt < TPW; tt++) {
            const int r = 16 * (TPW * w + tt) + n;
            uint32_t wd[8];
#pragma unroll
            for (int bs = 0; bs < 8; bs++)
                wd[bs] = *reinterpret_cast<const uint32_t *>(cur + T::QS + 16 * (8 * r + (bs ^ (n & 7))) + 4 * g);
            cw[tt].a = (u32x4){wd[0], wd[1], wd[2], wd[3]};
            cw[tt].b = (u32x4){wd[4], wd[5], wd[6], wd[7]};
            const u32x4 h = *reinterpret_cast<const u32x4 *>(cur + T::HDR + 16 * r);
#pragma unroll
            for (int bs = 0; bs < 8; bs++) ds[tt][bs] = f16_to_f32((uint16_t)(h[bs >> 1] >> (16 * (bs & 1))));
        }
        float accb[TPW][4];
#pragma unroll
        for (int tt = 0; tt < TPW; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) accb[tt][r] = 0.0f;
#pragma unroll
        for (int bs = 0; bs < 8; bs++) {
            const v8h ah = reinterpret_cast<const v8h *>(cur)[64 * bs + lane];
            const v8h al = reinterpret_cast<const v8h *>(cur + R16_PLANE)[64 * bs + lane];
#pragma unroll
            for (int tt = 0; tt < TPW; tt++) {
                const v8h q = r16_codes(cw[tt], k, bs, k6464);
                v4f Db = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, q, zero, 0, 0, 0);
                Db = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, q, Db, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) accb[tt][r] = fmaf(ds[tt][bs], Db[r], accb[tt][r]);
            }
        }
        const int4 e4 = reinterpret_cast<const int4 *>(cur + R16_EXO)[g];  // rows 4g .. 4g + 3
        const int ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
        for (int tt = 0; tt < TPW; tt++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[tt][r] = acc[tt][r] + ldexpf(accb[tt][r], ev[r]);
        if (tid < 16) badrow |= reinterpret_cast<const int *>(cur + R16_BADO)[tid];
    };
    auto compute = [&](const uint8_t *cur) {
        if constexpr (DT == kQ4) {
            compute_q4(cur);
            return;
        }
        R16W cw[TPW];
        R16K k[TPW];
#pragma unroll
        for (int tt = 0; tt < TPW; tt++) {
            const int r = 16 * (TPW * w + tt) + n;  // r % 8 == n % 8
            cw[tt].a = *reinterpret_cast<const u32x4 *>(cur + T::QS + 16 * (8 * r + (g ^ (n & 7))));
            cw[tt].b = *reinterpret_cast<const u32x4 *>(cur + T::QS + 16 * (8 * r + ((4 + g) ^ (n & 7))));
            cw[tt].h = *reinterpret_cast<const u32x4 *>(cur + T::HDR + 16 * r);
            r16_consts(k[tt], cw[tt], g);
        }
        v4f D[TPW];
#pragma unroll
        for (int tt = 0; tt < TPW; tt++) D[tt] = zero;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const v8h ah = reinterpret_cast<const v8h *>(cur)[64 * s + lane];
            const v8h al = reinterpret_cast<const v8h *>(cur + R16_PLANE)[64 * s + lane];
            v8h q[TPW];
#pragma unroll
            for (int tt = 0; tt < TPW; tt++) q[tt] = r16_codes(cw[tt], k[tt], s, k6464);
#pragma unroll
            for (int tt = 0; tt < TPW; tt++) D[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, q[tt], D[tt], 0, 0, 0);
#pragma unroll
            for (int tt = 0; tt < TPW; tt++) D[tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, q[tt], D[tt], 0, 0, 0);
        }
        const v4h xa = reinterpret_cast<const v4h *>(cur + R16_XSO)[lane];
        const int4 e4 = reinterpret_cast<const int4 *>(cur + R16_EXO)[g];  // rows 4g .. 4g + 3
        const int ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
        for (int tt = 0; tt < TPW; tt++) {
            const v4f mn = __builtin_amdgcn_mfma_f32_16x16x16f16(xa, k[tt].mB, zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float tv = k[tt].d * D[tt][r];
                tv = fmaf(-k[tt].dmin, mn[r], tv);
                acc[tt][r] = acc[tt][r] + ldexpf(tv, ev[r]);
            }
        }
        if (tid < 16) badrow |= reinterpret_cast<const int *>(cur + R16_BADO)[tid];
    };
    // Step for block b in stage `cur`: wait until this thread's loads of block b have landed (those of the next
    // block may still be in flight), barrier (everyone's have; nobody reads the stage of block b - 1 any more),
    // request block b + 2 into that stage, compute block b.
    // (a plain s_barrier: __syncthreads() would also wait for every load in flight, the next block's included)
    auto step = [&](const uint8_t *cur, uint8_t *nxt, int b) {
        R16_VMCNT(T::DMAS);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        stage(nxt, last(b + 2));
        compute(cur);
    };
    stage(st0, last(c0));
    stage(st1, last(c0 + 1));
    int b = c0;
    for (; b + 3 <= c1; b += 3) {
        step(st0, st2, b);
        step(st1, st0, b + 1);
        step(st2, st1, b + 2);
    }
    if (b < c1) step(st0, st2, b);
    if (b + 1 < c1) step(st1, st0, b + 1);
    R16_VMCNT(0);  // no DMA may still write LDS when the workgroup ends
    if (tid < 16) rowbad[tid] = badrow;
    __syncthreads();

    // results: straight to c with one slice, else the slice's partial tile [16][R]. Partials pass between
    // workgroups as agent-scope atomic stores and loads, which the L2 of each XCD does not hold back; each thread
    // waits for its stores to complete before the workgroup counts itself in, so the workgroup that counts last
    // sees every slice without a cache write-back or invalidation.
    const bool direct = !SWI && S == 1;
    float *pp = direct ? nullptr : part + ((rt * S + sl) * 16) * (int64_t)R;
    auto put = [&](int i, float v) {
        if (S > 1)
            __hip_atomic_store(pp + i, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            pp[i] = v;
    };
    auto get = [&](const float *q) -> float {
        return S > 1 ? __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *q;
    };
#pragma unroll
    for (int tt = 0; tt < TPW; tt++) {
        const int nl = 16 * (TPW * w + tt) + n;
        if (!row_ok(nl)) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 4 * g + r;
            if (m >= M || rowbad[m]) continue;
            if (direct) {
                cput(m * N + rt * R + nl, acc[tt][r]);
            } else {
                put(m * R + nl, acc[tt][r]);
            }
        }
    }
    int anybad = 0;
#pragma unroll
    for (int m = 0; m < 16; m++) anybad |= rowbad[m];
    if (anybad) {
        // rows holding NaN / Inf: exact float dot products over this slice in sdot32 order, on 32 lanes per output
        // (lane l runs chain l, elements k = l mod 32; then the fixed tree (a_l + a_l+8) + (a_l+16 + a_l+24),
        // s_l = Y_l + Y_l+4, (s_0 + s_2) + (s_1 + s_3) over shuffles), so the fallback adds no registers
        const int hl = lane >> 5, l32 = lane & 31;
        for (int i = 2 * w + hl; i < 16 * R; i += 8) {
            const int m = i / R, nl = i % R;
            const bool act = m < M && rowbad[m] && row_ok(nl);
            float a = 0.0f;
            if (act) {
                const int64_t row = row0 + out_row(nl);
                for (int64_t k = 256 * (int64_t)c0; k < 256 * (int64_t)c1; k += 32)
                    a = fmaf(xat(m * K + k + l32), deq_at<DT>(p, row, k + l32), a);
            }
            float v = a + __shfl_xor(a, 8);
            v = v + __shfl_xor(v, 16);
            v = v + __shfl_xor(v, 4);
            v = v + __shfl_xor(v, 2);
            v = v + __shfl_xor(v, 1);
            if (act && l32 == 0) {
                if (direct) {
                    cput(m * N + rt * R + nl, v);
                } else {
                    put(m * R + nl, v);
                }
            }
        }
    }
    if (direct) return;
    if (S > 1) {  // the workgroup that completes the row tile sums it
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (tid == 0)
            lastflag = __hip_atomic_fetch_add(&arrivals[rt], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        (uint32_t)(S - 1);
        __syncthreads();
        if (!lastflag) return;
        if (tid == 0) __hip_atomic_store(&arrivals[rt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        __syncthreads();
    }
    const float *base = part + (rt * S) * 16 * (int64_t)R;
    const int64_t stride = 16 * (int64_t)R;
    if (!SWI) {
        // thread i: partial elements 4 i .. 4 i + 3 (one row m, four consecutive columns), up to 8 slices in flight
        for (int i = tid; i < 4 * R; i += R16_THREADS) {
            const int m = (4 * i) / R, nl = (4 * i) % R;
            if (m >= M) continue;
            float sv[4];
#pragma unroll
            for (int e = 0; e < 4; e++) sv[e] = get(base + 4 * i + e);
            for (int k0 = 1; k0 < S; k0 += 8) {
                float v[8][4];
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (k0 + u < S)
#pragma unroll
                        for (int e = 0; e < 4; e++) v[u][e] = get(base + (k0 + u) * stride + 4 * i + e);
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (k0 + u < S)
#pragma unroll
                        for (int e = 0; e < 4; e++) sv[e] = sv[e] + v[u][e];
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (rt * R + nl + e >= N) break;
                cput(m * N + rt * R + nl + e, sv[e]);
            }
        }
    } else {
        // thread i: gate elements 4 i .. 4 i + 3 of the tile's first half and the up elements H further on
        for (int i = tid; i < 2 * R; i += R16_THREADS) {
            const int m = (4 * i) / H, il = (4 * i) % H;
            if (m >= M) continue;
            const int og = m * R + il, ou = og + H;
            float gv[4], uv[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                gv[e] = get(base + og + e);
                uv[e] = get(base + ou + e);
            }
            for (int k0 = 1; k0 < S; k0 += 4) {
                float vg[4][4], vu[4][4];
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (k0 + u < S)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            vg[u][e] = get(base + (k0 + u) * stride + og + e);
                            vu[u][e] = get(base + (k0 + u) * stride + ou + e);
                        }
#pragma unroll
                for (int u = 0; u < 4; u++)
                    if (k0 + u < S)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            gv[e] = gv[e] + vg[u][e];
                            uv[e] = uv[e] + vu[u][e];
                        }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (rt * H + il + e >= I) break;
                c[m * I + rt * H + il + e] = silu_ref(gv[e]) * uv[e];
            }
        }
    }
}

template <int DT, int TPW>
int run_rows16(trhip_ctx *ctx, const Planes &pl, int64_t nrows, int64_t N, int64_t row0, int64_t M, int64_t K,
               const void *x, const uint8_t *rec, int64_t RT, int S, int bps, void *c, float *part, bool acc,
               bool swi, int io) {
    const dim3 grid((unsigned)(RT * S)), block(R16_THREADS);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, 0, ctx->stream, pl, nrows, N, row0, M, K, x, rec, RT, S, bps, c, part,
                           ctx->arrivals);
        return launch_check(ctx, "rows16_gemm");
    };
    if (swi) return go(rows16_gemm<kQ4K, TPW, false, true>);
    if (io == TRHIP_F16) return acc ? go(rows16_gemm<DT, TPW, true, false, TRHIP_F16>) : go(rows16_gemm<DT, TPW, false, false, TRHIP_F16>);
    if (io == TRHIP_BF16) return acc ? go(rows16_gemm<DT, TPW, true, false, TRHIP_BF16>) : go(rows16_gemm<DT, TPW, false, false, TRHIP_BF16>);
    return acc ? go(rows16_gemm<DT, TPW, true, false>) : go(rows16_gemm<DT, TPW, false, false>);
}

}  // namespace

int launch_rows16(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                  int64_t M, bool acc, float *swi, int io) {
    const int dt = w->dtype;
    if ((dt != kQ4K && dt != kQ4) || M < 1 || M > 16 || w->K <= 0 || w->K % 256 != 0) return -1;
    if (dt == kQ4 && swi) return -1;  // the gate is fused for q4_k only
    if (swi && io != TRHIP_F32) return -1;
    const size_t xel = io == TRHIP_F32 ? sizeof(float) : sizeof(uint16_t);
    const int64_t K = w->K, nb = K / 256;
    const bool fused = swi != nullptr;
    if (fused && (N % 2 != 0 || acc)) return -1;
    const int64_t rows = fused ? N / 2 : N;  // output columns
    // tiles per wave and K slices: about two workgroups per CU, slices no shorter than one block. Chosen from the
    // store rows N alone, so the fused SwiGLU call splits K exactly as the plain call over the same store does.
    int tpw, S;
    if (ctx->force_rows16) {
        tpw = ctx->force_rows16 / 100 % 10;
        S = ctx->force_rows16 % 100;
    } else {  // one workgroup per CU, at most four slices (measured on the Llama shapes at M = 16)
        // 128-row tiles where they still give three workgroups for four CUs: each block's activation record then
        // serves twice the weight rows (28672x4096, M = 16, cold: 23.6 against 26.6 us; at 14336 rows the 112
        // workgroups take 21.8 against 16.7). Further K slices cost their partial sums: 14336x4096 in two slices
        // 19.4 against 16.7 us.
        // The slices are as many as fit one workgroup per CU: 6144x4096 in two slices (192 workgroups) 13.1 against
        // 15.9 us in three (288).
        const int64_t cus = ctx->sm_count > 0 ? ctx->sm_count : 256;
        tpw = 4 * ((N + 127) / 128) >= 3 * cus ? 2 : 1;
        const int64_t rt = (N + 64 * tpw - 1) / (64 * tpw);
        S = (int)(cus / rt);
        if (S > 4) S = 4;
    }
    if (S > nb) S = (int)nb;
    if (S < 1) S = 1;
    const int bps = (int)((nb + S - 1) / S);
    S = (int)((nb + bps - 1) / bps);
    const int64_t R = 64 * tpw, RT = fused ? (rows + R / 2 - 1) / (R / 2) : (rows + R - 1) / R;
    if (S > 1 && RT > trhip_ctx::kArrivalSlots) return -1;
    // the weight DMAs address a plane with 32-bit offsets
    if (w->N * nb * 128 > (int64_t)UINT32_MAX) return -1;
    // the record kernel reads x 16 bytes (fp32) or 8 bytes (16-bit) at a time
    const bool copy_x = reinterpret_cast<uintptr_t>(x) % (io == TRHIP_F32 ? 16 : 8) != 0;
    auto al = [](size_t v) { return (v + 255) / 256 * 256; };
    const size_t o_x = 0, o_r = al(copy_x ? (size_t)(M * K) * xel : 0);
    const size_t o_p = al(o_r + (size_t)nb * R16_XREC);
    const bool need_part = fused || S > 1;
    const size_t total = o_p + (need_part ? (size_t)(RT * S * 16 * R) * sizeof(float) : 0);
    int st = TRHIP_OK;
    uint8_t *ws = static_cast<uint8_t *>(workspace(ctx, total, &st));
    if (!ws) return st;
    const void *xa = x;
    if (copy_x) {
        hipError_t e = hipMemcpyAsync(ws + o_x, x, (size_t)(M * K) * xel, hipMemcpyDeviceToDevice, ctx->stream);
        if (e != hipSuccess) return hip_fail(ctx, e, "rows16: align x");
        xa = ws + o_x;
    }
    uint8_t *rec = ws + o_r;
    const dim3 rg((unsigned)nb), rb(R16_THREADS);
    auto rec_go = [&](auto kern) { hipLaunchKernelGGL(kern, rg, rb, 0, ctx->stream, xa, M, K, rec); };
    if (io == TRHIP_F16) dt == kQ4 ? rec_go(halves16_kernel<kQ4, TRHIP_F16>) : rec_go(halves16_kernel<kQ4K, TRHIP_F16>);
    else if (io == TRHIP_BF16) dt == kQ4 ? rec_go(halves16_kernel<kQ4, TRHIP_BF16>) : rec_go(halves16_kernel<kQ4K, TRHIP_BF16>);
    else dt == kQ4 ? rec_go(halves16_kernel<kQ4>) : rec_go(halves16_kernel<kQ4K>);
    if ((st = launch_check(ctx, "halves16")) != TRHIP_OK) return st;
    float *part = need_part ? reinterpret_cast<float *>(ws + o_p) : nullptr;
    void *dst = fused ? static_cast<void *>(swi) : c;
    const Planes pl = w->planes();
    if (dt == kQ4)
        return tpw == 2 ? run_rows16<kQ4, 2>(ctx, pl, w->N, N, row0, M, K, xa, rec, RT, S, bps, dst, part, acc, false, io)
                        : run_rows16<kQ4, 1>(ctx, pl, w->N, N, row0, M, K, xa, rec, RT, S, bps, dst, part, acc, false, io);
    if (tpw == 2) return run_rows16<kQ4K, 2>(ctx, pl, w->N, N, row0, M, K, xa, rec, RT, S, bps, dst, part, acc, fused, io);
    return run_rows16<kQ4K, 1>(ctx, pl, w->N, N, row0, M, K, xa, rec, RT, S, bps, dst, part, acc, fused, io);
}

}  // namespace trhip
