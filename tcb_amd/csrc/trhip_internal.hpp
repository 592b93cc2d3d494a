// trhip_internal.hpp -- shared definitions of libtrhip (gfx950 only).
//
// Device layout of a weight store ("planes"). GGUF blocks are uploaded unchanged and then
// repacked on the device, field by field, so that every plane is 16-byte aligned and a lane's
// bytes for one block are contiguous. Nothing is decoded; the repack is a byte permutation and
// trhip_wstore_to_raw inverts it exactly. Per row of nb blocks:
//
//   q8   : qs [N][nb][32]  int8 codes (block order)          d [N][nb] fp16
//   q4   : qs [N][nb][16]  packed nibbles (block order)       d [N][nb] fp16
//   q4_k : hdr[N][nb][16]  d, dmin, scales[12] (block order)  qs[N][nb][128] lane-sliced (see below)
//   q6_k : ql [N][nb][128] lane-sliced   qh [N][nb][64] lane-sliced   sc [N][nb][16]   d [N][nb] fp16
//
// Lane slicing. q4_k qs: the factored GEMV gives lane (g, h) of a row bytes 32g + 16h .. +16 of every
// block (low and high nibbles: 16 elements each of sub-blocks 2g and 2g+1); the exact GEMV gives lane
// t bytes 32g + 8t .. +8 for every g (it owns sdot32 accumulator t, tensor/cpu_gemv_amd64.s:190-213).
// With 8-byte pieces C(g, t) = old[32g + 8t, +8) stored at 16-byte-slot 4(t>>1) + g, half t&1, the
// factored lane reads one contiguous 16-byte slice and the exact lane four 8-byte pieces:
//   q4_k qs  : new[64(t>>1) + 16g + 8(t&1) + l] = old[32g + 8t + l]    (g, t < 4, l < 8)
// q6_k (exact GEMV lane t owns elements 8t..8t+7 of every 32-element group):
//   q6_k ql  : new[32t + 16n + 8h + l]  = old[64n + 32h + 8t + l]      (n, h < 2, l < 8)
//   q6_k qh  : new[16t + 8n + l]        = old[32n + 8t + l]            (n < 2, l < 8)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/trhip.h"

namespace trhip {

constexpr int kQ8 = TRHIP_Q8, kQ4 = TRHIP_Q4, kQ4K = TRHIP_Q4K, kQ6K = TRHIP_Q6K;

__host__ __device__ constexpr int block_elems(int dt) { return (dt == kQ8 || dt == kQ4) ? 32 : 256; }
__host__ __device__ constexpr int block_bytes(int dt) {  // tensor/quant.go:23-29
    return dt == kQ8 ? 34 : dt == kQ4 ? 18 : dt == kQ4K ? 144 : 210;
}

// Planes of one store (all pointers are device pointers into one allocation).
struct Planes {
    const uint8_t *qs;   // q8/q4 codes, q4_k qs, q6_k ql
    const uint8_t *aux;  // q4_k hdr, q6_k qh
    const uint8_t *sc;   // q6_k scales
    const uint16_t *d;   // q8/q4/q6_k fp16 scale
    int64_t nb;          // blocks per row
};

// Bytes per block in each plane.
__host__ __device__ constexpr int qs_bytes(int dt) { return dt == kQ8 ? 32 : dt == kQ4 ? 16 : 128; }
__host__ __device__ constexpr int aux_bytes(int dt) { return dt == kQ4K ? 16 : dt == kQ6K ? 64 : 0; }
__host__ __device__ constexpr int sc_bytes(int dt) { return dt == kQ6K ? 16 : 0; }
__host__ __device__ constexpr int d_bytes(int dt) { return dt == kQ4K ? 0 : 2; }

// Position in a repacked q4_k qs block of original qs byte i = 32g + 8t + l.
__host__ __device__ constexpr int q4k_pos(int i) {
    return 64 * ((i >> 4) & 1) + 16 * (i >> 5) + 8 * ((i >> 3) & 1) + (i & 7);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {  // exact for finite values and +-Inf
    return (float)__builtin_bit_cast(_Float16, h);
}

// 16-bit activation / output formats of the typed entry point (TRHIP_F16, TRHIP_BF16), widened and rounded as the
// reference does. Widening is exact: bf16ToF32 (tensor/cpu_dtype.go:83), f16ToF32 (:125-145, a NaN keeps its
// payload). Rounding to nearest even with the reference's NaN and overflow rules: f32ToBF16 (:73-80, NaN quieted by
// or-ing 0x0040), f32ToF16 (:87-123, NaN quieted as 0x7E00 | payload >> 13; 65520 and above to Inf; subnormals
// rounded from the shifted significand).
__device__ __forceinline__ float h16_to_f32(uint32_t h, int io) {
    if (io == TRHIP_BF16) return __uint_as_float(h << 16);
    // finite values (subnormals included) convert exactly in hardware; Inf / NaN keep their bits as the reference
    // widens them (the payload shifted up, no quieting): a select, not a branch
    const float v = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    const float s = __uint_as_float(((h & 0x8000u) << 16) | 0x7F800000u | ((h & 0x3FFu) << 13));
    return ((h >> 10) & 0x1Fu) == 0x1Fu ? s : v;
}
// f32 -> bf16 / f16, rounded to nearest even (tensor/cpu_dtype.go:73-123). f16: the hardware conversion rounds
// finite values to nearest even, subnormal results and overflow to Inf included, as the reference does; a NaN is
// sign | 0x7E00 | (mantissa >> 13) in the reference, chosen by a select.
__device__ __forceinline__ uint32_t f32_to_h16(float f, int io) {
    uint32_t b = __float_as_uint(f);
    if (io == TRHIP_BF16) {
        const uint32_t nan = ((b >> 16) | 0x0040u) & 0xFFFFu;
        const uint32_t r = (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
        return (b & 0x7FFFFFFFu) > 0x7F800000u ? nan : r;
    }
    const uint32_t hw = __builtin_bit_cast(uint16_t, (_Float16)f);
    const uint32_t nan = ((b >> 16) & 0x8000u) | 0x7E00u | ((b & 0x7FFFFFu) >> 13);
    return (b & 0x7FFFFFFFu) > 0x7F800000u ? nan : hw;
}

// Hide a value from the optimizer (no instruction is emitted). Used on a dword-wide nibble mask so the
// compiler keeps one v_and_b32 per four codes and converts each byte with one v_cvt_f32_ubyte{k},
// instead of folding the mask into four per-byte bit-field extracts.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}
// The same without volatile: the value stays hidden, but the (empty) statement has no side effects, so the
// scheduler may still move loads across it (a volatile one keeps every LDS read of a loop body in program order,
// each waited for where it is used).
__device__ __forceinline__ uint32_t hide(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

// Global -> LDS copies (buffer_load ... lds) issued as inline assembly. The compiler's waitcnt pass, when it sees
// an LDS-DMA request in flight, makes every later LDS access it cannot prove disjoint from the request's destination
// wait for all requests (vmcnt(0)), which turns a prefetch into a stall. Issued this way the requests are invisible
// to it: the caller waits for them itself with s_waitcnt vmcnt (they complete in issue order), and must not let
// compiler-visible vector memory loads be outstanding behind them (the compiler's own wait for such a load would
// count only its loads).
//
// Buffer descriptor over [base, base + bytes): per-lane 32-bit offsets; a load past the end reads zeros.
typedef uint32_t dma_rsrc __attribute__((ext_vector_type(4)));
__device__ __forceinline__ dma_rsrc dma_desc(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    return (dma_rsrc){(uint32_t)a, (uint32_t)(a >> 32) & 0xFFFFu, bytes, 0x00020000u};
}
// LDS address of a __shared__ pointer (wave-uniform destinations go in M0).
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)reinterpret_cast<uintptr_t>(p); }
// 16 bytes per lane from r at voff + soff into LDS at dst + 16 * lane (dst wave-uniform).
__device__ __forceinline__ void dma16(dma_rsrc r, uint32_t dst, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(dst), "v"(voff), "s"(r), "s"(soff)
                 : "memory", "m0");
}
// 4 bytes per lane into LDS at dst + 4 * lane.
__device__ __forceinline__ void dma4(dma_rsrc r, uint32_t dst, uint32_t voff, uint32_t soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                 :
                 : "s"(dst), "v"(voff), "s"(r), "s"(soff)
                 : "memory", "m0");
}
// s_waitcnt vmcnt(n) for n known once the caller's loop is unrolled (the switch folds to one instruction).
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
#define TRHIP_VMW(k) \
    case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        TRHIP_VMW(0) TRHIP_VMW(1) TRHIP_VMW(2) TRHIP_VMW(3) TRHIP_VMW(4) TRHIP_VMW(5) TRHIP_VMW(6) TRHIP_VMW(7)
        TRHIP_VMW(8) TRHIP_VMW(9) TRHIP_VMW(10) TRHIP_VMW(11) TRHIP_VMW(12) TRHIP_VMW(13) TRHIP_VMW(14)
        TRHIP_VMW(15) TRHIP_VMW(16) TRHIP_VMW(17) TRHIP_VMW(18) TRHIP_VMW(19) TRHIP_VMW(20) TRHIP_VMW(21)
        TRHIP_VMW(22) TRHIP_VMW(23) TRHIP_VMW(24) TRHIP_VMW(25) TRHIP_VMW(26) TRHIP_VMW(27) TRHIP_VMW(28)
        TRHIP_VMW(29) TRHIP_VMW(30) TRHIP_VMW(31)
#undef TRHIP_VMW
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    }
}
// Workgroup barrier for data exchanged through LDS: this wave's LDS accesses complete, then s_barrier. (The release
// fence of __syncthreads also waits for every outstanding vector memory request.)
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// First v_dot4_i32_i8 of a chain (sum of the four signed byte products plus c) in its three-operand form, whose
// result register is not the accumulator. __builtin_amdgcn_sdot4 is emitted as the two-operand v_dot4c, which
// accumulates in place, so a chain started from 0 or from a value still needed later costs a v_mov first.
__device__ __forceinline__ int sdot4_zero(int a, int b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ int sdot4_from(int a, int b, int c) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Byte k (0..3) of a dword as float: v_cvt_f32_ubyte{k}.
__device__ __forceinline__ float ubyte_f(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xFFu); }

// q4_k scale/min unpack for all 8 sub-blocks from the 12 scale bytes (tensor/quant.go:158-163),
// done four bytes at a time. sc[j], m[j] are returned as 4 packed bytes each (j < 4, j >= 4).
__device__ __forceinline__ void q4k_scales(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t &sc_lo,
                                           uint32_t &sc_hi, uint32_t &m_lo, uint32_t &m_hi) {
    sc_lo = s0 & 0x3F3F3F3Fu;
    m_lo = s1 & 0x3F3F3F3Fu;
    sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    m_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
}

// Element k of weight row `row`, dequantized exactly as tensor/quant.go:139-205 (scalar, slow;
// used where one element at a time is needed).
template <int DT>
__device__ __forceinline__ float deq_at(const Planes p, int64_t row, int64_t k) {
    constexpr int be = block_elems(DT);
    int64_t bi = row * p.nb + k / be;
    int e = (int)(k % be);
    if (DT == kQ8) {
        return (float)(int8_t)p.qs[bi * 32 + e] * f16_to_f32(p.d[bi]);
    } else if (DT == kQ4) {
        uint8_t b = p.qs[bi * 16 + (e & 15)];
        int code = (e < 16) ? (b & 0xF) : (b >> 4);
        return (float)(code - 8) * f16_to_f32(p.d[bi]);
    } else if (DT == kQ4K) {
        const uint8_t *h = p.aux + bi * 16;
        int j = e >> 5, g = e >> 6, ee = e & 31;
        const uint8_t *s = h + 4;
        uint8_t scv, mv;
        if (j < 4) { scv = s[j] & 63; mv = s[j + 4] & 63; }
        else { scv = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)); mv = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4)); }
        float d = f16_to_f32((uint16_t)(h[0] | (h[1] << 8))), dmin = f16_to_f32((uint16_t)(h[2] | (h[3] << 8)));
        uint8_t b = p.qs[bi * 128 + q4k_pos(32 * g + ee)];
        int code = (j & 1) ? (b >> 4) : (b & 0xF);
        return (d * (float)scv) * (float)code - dmin * (float)mv;
    } else {
        int n = e >> 7, k4 = (e >> 5) & 3, ee = e & 31;
        uint8_t lo = p.qs[bi * 128 + 32 * (ee >> 3) + 16 * n + 8 * (k4 & 1) + (ee & 7)];
        uint8_t hb = p.aux[bi * 64 + 16 * (ee >> 3) + 8 * n + (ee & 7)];
        int nib = (k4 < 2) ? (lo & 0xF) : (lo >> 4);
        int code = nib | (((hb >> (2 * k4)) & 3) << 4);
        int8_t scv = (int8_t)p.sc[bi * 16 + 8 * n + 2 * k4 + ee / 16];
        return f16_to_f32(p.d[bi]) * (float)scv * (float)(code - 32);
    }
}

// silu(x) = x sigma(x) as TR's siluForward (tensor/cpu_elementwise_wide.go:101-116, sigmoidBlock :83-98) with e^x
// the AVX2 expVec it runs for every element (tensor/cpu_vector_amd64.s:13-38): clamp to [-104, 89] (NaN takes the
// lower bound and is put back at the end), n = rne(x log2e), r = x - n ln2 in two fused steps (ln2 split high/low),
// a degree-6 polynomial in fused steps, and 2^n applied as 2^(n>>1) * 2^(n - n>>1), so subnormal results and
// overflow to +Inf come out right. Same operations in the same order (files are built with -ffp-contract=off).
__device__ __forceinline__ float exp_ref(float x) {
    float x1 = x > -104.0f ? x : -104.0f;
    x1 = x1 < 89.0f ? x1 : 89.0f;
    const float n = __builtin_rintf(x1 * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693359375f, x1);
    r = __builtin_fmaf(-n, -2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    const float z = r * r;
    p = __builtin_fmaf(z, p, r);
    float y = p + 1.0f;
    const int ni = (int)n, h = ni >> 1, l = ni - h;
    y = y * __builtin_bit_cast(float, (uint32_t)(h + 127) << 23);
    y = y * __builtin_bit_cast(float, (uint32_t)(l + 127) << 23);
    return x != x ? x : y;
}
// x sigma(x) with e = e^-|x|: sigma = 1/(1+e) for x >= 0, e/(1+e) otherwise; sigma == 0 gives +0.
__device__ __forceinline__ float silu_ref(float x) {
    const float e = exp_ref(-__builtin_fabsf(x));
    const float s = x >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    return (s == 0.0f ? 0.0f : x) * s;
}

// Exact fp32 dot of activation row xr with weight row `row` over elements [k0, k1) (multiples of 32) in sdot32
// order (fallback for rows with NaN/Inf; one thread, 32 chains).
template <int DT>
__device__ __forceinline__ float exact_dot_range(const Planes p, int64_t row, const float *__restrict__ xr, int64_t k0,
                                                 int64_t k1) {
    float acc[32];
#pragma unroll
    for (int l = 0; l < 32; l++) acc[l] = 0.0f;
    for (int64_t k = k0; k < k1; k += 32)
#pragma unroll
        for (int l = 0; l < 32; l++) acc[l] = fmaf(xr[k + l], deq_at<DT>(p, row, k + l), acc[l]);
    float Y[8];
#pragma unroll
    for (int l = 0; l < 8; l++) Y[l] = (acc[l] + acc[8 + l]) + (acc[16 + l] + acc[24 + l]);
    float s0 = Y[0] + Y[4], s1 = Y[1] + Y[5], s2 = Y[2] + Y[6], s3 = Y[3] + Y[7];
    return (s0 + s2) + (s1 + s3);
}
template <int DT>
__device__ __forceinline__ float exact_dot_row(const Planes p, int64_t row, const float *__restrict__ xr, int64_t K) {
    return exact_dot_range<DT>(p, row, xr, 0, K);
}

// Tiled activation layout of the q4_k prefill kernel (prefill.hip), per 32-row tile mt = m / 32 and block b, in
// the operand order of its MFMAs so that each 1 KB piece is one coalesced load straight into LDS:
//   codes   : 8 KB = chunk kc (32 elements of sub-block kc) x lane (r + 32 h) x 16 bytes (elements 32 kc + 16 h + i)
//   msum    : 1 KB = lane (r + 32 half) x 8 f16: half 0 = Sh_0..7, half 1 = Sl_0..7 (S_j = 64 Sh_j + Sl_j)
//   scales  : 32 floats d8 of rows r
// Rows are padded to a multiple of 128 (a workgroup's row tile); pad rows hold no meaningful values.
__host__ __device__ inline int64_t tiled_q(int64_t m, int64_t b, int64_t nb, int k) {
    return (((m >> 5) * nb + b) * 8 + (k >> 5)) * 1024 + ((m & 31) + 32 * ((k >> 4) & 1)) * 16 + (k & 15);
}
__host__ __device__ inline int64_t tiled_d(int64_t m, int64_t b, int64_t nb) { return ((m >> 5) * nb + b) * 32 + (m & 31); }
__host__ __device__ inline int64_t tiled_sj(int64_t m, int64_t b, int64_t nb, int half, int j) {  // in f16 units
    return ((m >> 5) * nb + b) * 512 + ((m & 31) + 32 * half) * 8 + j;
}
constexpr int64_t kPrefillRowPad = 128;

}  // namespace trhip


struct trhip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    // Grow-only device workspace (activation copies, quantized activations).
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // A second one for results an entry point keeps while it calls another that uses the first
    // (the merged gate_up output of trhip_gemm_q_swiglu).
    void *ws2 = nullptr;
    size_t ws2_bytes = 0;
    // A third for the fp32 copies of 16-bit activations and outputs (trhip_gemm_q_typed), which live across the call
    // of the fp32 operator that uses the others.
    void *ws3 = nullptr;
    size_t ws3_bytes = 0;
    // Workspace buffers replaced by a larger one while instantiated graphs of this context exist: their kernel
    // nodes may still hold the old addresses, so the buffers are freed only when the last graph is destroyed
    // (or with the context).
    std::vector<void *> retired;
    int live_graphs = 0;
    // Weight stores of this context not yet destroyed: each holds the context's stream, so the context refuses to
    // be destroyed before them (and before its graphs).
    int live_stores = 0;
    // Pinned host staging for host-side index arrays (trhip_embedding_q): reused once the copy that last read it
    // has completed (idx_done).
    void *idx_host = nullptr;
    size_t idx_host_bytes = 0;
    hipEvent_t idx_done = nullptr;
    // Pinned host ring for chunked weight uploads (trhip_wstore_create): UP_SLOTS buffers of up_slot_bytes,
    // slot s reusable once up_done[s] (recorded after its host-to-device copy) has completed.
    static constexpr int UP_SLOTS = 2;
    void *up_host[UP_SLOTS] = {nullptr, nullptr};
    void *up_dev[UP_SLOTS] = {nullptr, nullptr};
    hipEvent_t up_done[UP_SLOTS] = {nullptr, nullptr};
    size_t up_slot_bytes = 0;
    // Launch-shape overrides set by trhip_set_launch_shape (tests and tuning only); 0 = the built-in choice.
    int force_kl = 0;           // K-across-lanes GEMV: 1000 WAVES + 100 KS + 10 PD + RPW / 8
    int kl_min_wgs = 0;         // K-across-lanes GEMV: at least this many workgroups (0: built-in)
    int force_fast_q4k = 0;     // row-sliced fast q4_k GEMV: 1000 D + 100 WAVES + 10 KS + R
    int force_exact_rows = 0;   // exact four-lane GEMV rows per workgroup (16, 32, 64)
    int force_exact_lanes = 0;  // exact GEMV lanes per row (4, 8, 16)
    int force_actq_tm = 0;      // act-quant MFMA row tile (32, 64)
    int force_actq_slices = 0;  // act-quant MFMA K slices, fast mode (0: built-in)
    int force_rows16 = 0;       // batched-decode q4_k kernel: 100 tiles per wave + K slices
    // Arrival counters of kernels whose K slices are summed by the workgroup that finishes a row tile last
    // (rows16.hip): kArrivalSlots zeroed words, each returned to zero by that workgroup.
    static constexpr int64_t kArrivalSlots = 65536;
    uint32_t *arrivals = nullptr;
    // Device address of the static scratch array of trhip_gemm_q_actq_noalloc on this context's device.
    uint8_t *scratch = nullptr;
    int sm_count = 0;
};

struct trhip_wstore {
    trhip_ctx *ctx = nullptr;
    int dtype = 0;
    int64_t N = 0, K = 0, nb = 0;
    uint8_t *base = nullptr;  // one device allocation
    size_t bytes = 0;
    uint8_t *qs = nullptr, *aux = nullptr, *sc = nullptr;
    uint16_t *d = nullptr;
    trhip::Planes planes() const { return trhip::Planes{qs, aux, sc, d, nb}; }
};

namespace trhip {
// Error helpers (api.hip).
int fail(trhip_ctx *ctx, int code, const std::string &msg);
int hip_fail(trhip_ctx *ctx, hipError_t e, const char *what);
int launch_check(trhip_ctx *ctx, const char *what);
void *workspace(trhip_ctx *ctx, size_t bytes, int *status);
void *workspace2(trhip_ctx *ctx, size_t bytes, int *status);
// Allow `bytes` of dynamic LDS for kernel `fn` on the context's device (needed above 64 KB); done once per device
// and kernel, thread-safe.
int allow_dyn_lds(trhip_ctx *ctx, const void *fn, size_t bytes, const char *what);
// Whether the context's stream is being captured into a graph.
bool capturing(trhip_ctx *ctx);

// Kernel launchers (one per source file). All return TRHIP_OK or an error code.
// GGUF blocks [block0, block0 + nblocks) of the store, held in raw_dev from its start, into the planes.
int launch_repack(trhip_ctx *ctx, trhip_wstore *w, const uint8_t *raw_dev, int64_t block0, int64_t nblocks);
int launch_swiglu(trhip_ctx *ctx, const float *gu, int64_t M, int64_t I, float *out);
int launch_unpack(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t rows, uint8_t *raw_dev);
int launch_dequant(trhip_ctx *ctx, const trhip_wstore *w, int64_t block0, int64_t nblocks, float *out);
int launch_embedding(trhip_ctx *ctx, const trhip_wstore *w, const int64_t *idx, int64_t nidx, float *out,
                     int *bad_dev);
int launch_gemv(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                bool acc, int mode);
// Fast-mode GEMV over a merged [gate | up] store of 2I rows with the SwiGLU gate fused: out[i] = silu(g_i) * u_i,
// bit-identical to the fast GEMV followed by launch_swiglu. Returns -1 (nothing launched) where the fused kernel
// does not apply.
int launch_gemv_fast_swiglu(trhip_ctx *ctx, const trhip_wstore *w, const float *x, float *out, int64_t I);
int launch_gemm_rows(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                     int64_t M, bool acc);
// swi != nullptr (set, not accumulate; N = 2I rows [gate | up]): out swi[m, i] = silu(c[m, i]) * c[m, I + i], fused
// into the slice sum when K is split (c is then not written), else after it
int launch_gemm_rows_fast(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                          int64_t M, bool acc, float *swi = nullptr);
int launch_quantize_q8(trhip_ctx *ctx, const float *x, int64_t M, int64_t K, int blk, int8_t *q, float *d,
                       int16_t *bs, uint8_t *bad, uint16_t *sj);
int launch_read_probe(trhip_ctx *ctx, const void *p, int64_t bytes);
// The q4_k prefill path over the tiled activation layout: whether it takes (M, N), the tiled quantizer, the kernel.
bool prefill_tiles_apply(int dtype, int64_t M, int64_t N, int64_t row0, int64_t K);
int launch_quantize_tiles(trhip_ctx *ctx, const float *x, int64_t M, int64_t K, int8_t *qt, float *dt, uint16_t *st,
                          uint8_t *bad);
// fast: the same exact integer block sums with the fp32 epilogue fused (tolerance mode); else bit-exact.
int launch_prefill_q4k(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                       int64_t M, bool acc, const int8_t *qt, const float *dt, const uint16_t *st, const uint8_t *bad,
                       bool fast);
// q6_k weights on the same tiles (prefill.hip), always exact.
int launch_prefill_q6k(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                       int64_t M, bool acc, const int8_t *qt, const float *dt, const uint8_t *bad);
// 16-bit activations / outputs (io16.hip): dst[i] = widen(src[i]) and dst[i] = round(src[i]) for n elements.
int launch_widen16(trhip_ctx *ctx, const uint16_t *src, float *dst, int64_t n, int io);
int launch_round16(trhip_ctx *ctx, const float *src, uint16_t *dst, int64_t n, int io);
// The fast K-across-lanes GEMV reading 16-bit x and writing 16-bit c (io) directly (gemv_fast.hip), or -1 when the
// store's shape does not take that kernel.
int launch_gemv_fast_io(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                        bool acc, int io);
// The exact GEMV with 16-bit x (8-byte aligned) and c of one type (gemv.hip).
int launch_gemv_exact_io(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                         bool acc, int io);
void *workspace3(trhip_ctx *ctx, size_t bytes, int *status);

// The prefill kernels' inner loop alone on their real grid (prefill.hip): kind 0 q4_k exact, 1 q4_k fast, 2 q6_k.
int launch_prefill_probe(trhip_ctx *ctx, int kind, int64_t M, int64_t N, int64_t K);
int launch_mfma_probe(trhip_ctx *ctx, int valu_per_mfma, int waves_per_simd, int64_t iters);
// Fast-mode q4_k product for 1 <= M <= 16 activation rows in one launch (rows16.hip); swi as in
// launch_gemm_rows_fast. Returns -1 (nothing launched) where it does not apply.
// io: TRHIP_F32, or f16 / bf16 x and c (read and written directly; not with swi).
int launch_rows16(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, void *c,
                      int64_t M, bool acc, float *swi = nullptr, int io = TRHIP_F32);
// q4_0 and q6_k act-quant on int8 matrix cores (actq4.hip, actq6.hip): whether each takes the shape, and the kernel.
bool actq4_mfma_applies(int64_t M, int64_t N, int64_t row0, int64_t K);
int launch_actq4_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                      int64_t M, bool acc, const int8_t *q, const float *d, const uint8_t *bad);
bool actq6_mfma_applies(int64_t M, int64_t N, int64_t row0, int64_t K);
int launch_actq6_mfma(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                      int64_t M, bool acc, const int8_t *q, const float *d, const uint8_t *bad);
int launch_actq(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x, float *c,
                int64_t M, bool acc, const int8_t *q, const float *d, const int16_t *bs, const uint8_t *bad,
                const uint16_t *sj, bool fast);
}  // namespace trhip
