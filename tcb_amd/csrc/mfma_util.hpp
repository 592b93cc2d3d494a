// mfma_util.hpp -- helpers shared by the matrix-core kernels (actq_mfma.hip, prefill.hip): operand vector
// types, the two-plane weight expansion, f16 packing of small integers, tile row states and the XCD-aware
// workgroup-to-tile mapping.
#pragma once

#include "trhip_internal.hpp"

namespace trhip {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

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

// Row states of a tile of TM activation rows from per-(row, block) NaN/Inf flags flags[row * nb + b]:
// st[r] = 0 (finite), 1 (some block flagged) or 2 (row m0 + r is past M), *any = 1 if some row is 1. Every thread
// takes a share of the flags, so the loads are independent rather than one chain per row. Ends with a barrier.
template <int TM, int THREADS>
__device__ __forceinline__ void tile_row_flags(const uint8_t *__restrict__ flags, int64_t m0, int64_t M, int nb,
                                               int *st, int *any) {
    const int tid = threadIdx.x;
    if (tid < TM) st[tid] = m0 + tid < M ? 0 : 2;
    if (tid == 0) *any = 0;
    __syncthreads();
    constexpr int P = THREADS / TM;  // threads per row
    const int r = tid % TM, part = tid / TM;
    if (m0 + r < M) {
        const uint8_t *f = flags + (m0 + r) * nb;
        int v = 0;
#pragma unroll 8
        for (int b = part; b < nb; b += P) v |= f[b];
        if (v) {
            atomicOr(&st[r], 1);
            *any = 1;
        }
    }
    __syncthreads();
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

}  // namespace
}  // namespace trhip
