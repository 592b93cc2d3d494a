/*
 * trq_oracle.h -- CPU oracle for TR's quantized GGUF matmul (test infrastructure only).
 *
 * This is a plain-C restatement of the reference's CPU algorithm, used ONLY as the
 * expected result of the parity tests (tests/), __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 * The product (libtrhip) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to the
 * reference repository root, package internal/compute/tensor unless stated).
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   trq_f16_to_f32, trq_dequant       golden FNV-1a hashes of quant_test.go:63-66 + known values
 *   trq_check_quant_scales            TestCheckQuantScales table (quant_test.go:162-181)
 *   trq_quant_zero_raw                TestDequantKnownValues zero-constructor case (quant_test.go:117-126)
 *   trq_dot_f32                       hand-derived known answers for the sdot32 lane/tree order
 *                                     + bitwise agreement with trq_avx2_sdot32 (intrinsics that
 *                                     follow cpu_gemv_amd64.s:190-227 instruction by instruction)
 *   trq_quant_dot                     == dequant + dot_f32 by construction (dotQuantGo) and bitwise
 *                                     equal to the AVX2 restatements of sdotq8/q4/q4k/q6k
 *   trq_quant_gemm (M>1)              per-256-chunk order checked against a float64 bound and an
 *                                     independent numpy restatement of the chunk order
 *   trq_quantize_q8                   TestQuantizeQ8KEdgeBlocks / TestQuantizeQ8BlockEdges answers
 *   trq_dot_q4q8/_q4kq8/_q6kq8        integer parts vs brute-force int64 from dequantized codes;
 *                                     float epilogue vs the float64 closeness bound of
 *                                     cpu_quant_q8_test.go:84
 *   trq_round16 / trq_widen16         the reference's known answers (dtype_test.go:16-88), the round trip
 *                                     of every 16-bit pattern, numpy's IEEE float16 rounding, nearest-even
 *                                     bf16 by exhaustive neighbour comparison
 */
#ifndef TRQ_ORACLE_H
#define TRQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantized dtypes (names follow the reference: "q8", "q4", "q4_k", "q6_k"). */
enum { TRQ_Q8 = 1, TRQ_Q4 = 2, TRQ_Q4K = 3, TRQ_Q6K = 4 };

int trq_block_elems(int dt);
int trq_block_bytes(int dt);

/* cpu_dtype.go:126-145 (f16ToF32): exact, incl. subnormals and NaN payload. */
float trq_f16_to_f32(uint16_t h);
/* 16-bit activations and outputs, type 1 = float16, 2 = bfloat16: cpu_dtype.go:73-145 (rounding to nearest even,
 * NaN quieted; widening exact). */
void trq_round16(int type, const float *src, uint16_t *dst, size_t n);
void trq_widen16(int type, const uint16_t *src, float *dst, size_t n);

/* quant.go:158-163 (q4kScale). */
void trq_q4k_scale(int j, const uint8_t *scales12, uint8_t *sc, uint8_t *m);

/* quant.go:207-221 (dequantBlocks): nblocks whole blocks of raw -> y. */
void trq_dequant(int dt, const uint8_t *raw, size_t nblocks, float *y);

/* quant.go:108-128 (CheckQuantScales): index of first block with NaN/Inf scale, else -1. */
long trq_check_quant_scales(int dt, const uint8_t *raw, size_t nbytes);

/* quant.go:416-427 (QuantZeroRaw): bytes of n zero elements. */
void trq_quant_zero_raw(int dt, size_t n, uint8_t *out);

/* cpu_gemv_amd64.go:25-35 (dotF32) with sdot32 (cpu_gemv_amd64.s:190-227) and the
 * dot32 tail (cpu_gemv.go:66-85). */
float trq_dot_f32(const float *x, const float *y, size_t n);

/* cpu_quant.go:38-44 (dotQuantGo) == quantDot (cpu_quant_amd64.go:28-41). */
float trq_quant_dot(int dt, const float *x, const uint8_t *w, size_t K);

/* cpu_quant.go:47-83 (quantGemm) incl. quantGemv (:151) and quantGemmPanels (:103):
 * c[m,n] += sum_k a[m,k] * deq(w)[n,k]; a [M,K], w [N,K] blocks, c [M,N]. */
void trq_quant_gemm(int dt, size_t M, size_t N, size_t K, const float *a, const uint8_t *w,
                    float *c, int threads);

/* cpu_quant_q8.go:39-68 (quantizeQ8): q [K], d [K/blk], bs [K/16]. */
void trq_quantize_q8(const float *x, size_t K, int blk, int8_t *q, float *d, int16_t *bs);

/* cpu_quant_q8.go:74-87, :91-116, :378-407 (Go twins, explicitly rounded). */
float trq_dot_q4q8(size_t blocks, const uint8_t *w, const int8_t *q, const float *d);
float trq_dot_q4kq8(size_t blocks, const uint8_t *w, const int8_t *q, const float *d,
                    const int16_t *bs);
float trq_dot_q6kq8(size_t blocks, const uint8_t *w, const int8_t *q, const float *d,
                    const int16_t *bs);

/* Integer per-block sums of the act-quant kernels for one weight row and one activation
 * row: Q4_0 isum; Q4_K isum and msum; Q6_K the single integer (isum - 32*msum). */
void trq_block_isums(int dt, size_t blocks, const uint8_t *w, const int8_t *q, const int16_t *bs,
                     int32_t *isum, int32_t *msum);

/* cpu_quant_q8.go:125-134 (quantGemmAct) -> quantGemvQ8 (:159) / quantGemmQ8 (:186):
 * rows with NaN/Inf take the fp32 path (quantGemv) for that row only. */
void trq_quant_gemm_act(int dt, size_t M, size_t N, size_t K, const float *a, const uint8_t *w,
                        float *c, int threads);

/* cpu_quant.go:163-171 (quantEmbedding). */
void trq_quant_embedding(int dt, const uint8_t *raw, size_t D, const int64_t *idx, size_t nidx,
                         float *out);

/* quant_test.go:20-46 (randomQuant) and FNV-1a-64 over LE float32 bits (quant_test.go:72-77). */
void trq_random_quant(int dt, uint32_t seed, size_t blocks, uint8_t *out);
uint64_t trq_fnv1a64_f32(const float *y, size_t n);

/* SwiGLU epilogue: e^x as the reference's AVX2 expVec (cpu_vector_amd64.s:13-38), silu as siluForward
 * (cpu_elementwise_wide.go:101-116), and silu(g) * u over a [M, 2I] [G | U] buffer (lib/layers.tr:223). */
float trq_exp_vec(float x);
float trq_silu(float x);
void trq_swiglu(const float *gu, size_t M, size_t I, float *out);

/* AVX2/FMA/F16C restatements of the reference's assembly (trq_avx2.c): the CPU baseline.
 * They follow the .s instruction sequences and must agree bitwise with the scalar oracle. */
int trq_avx2_available(void);
float trq_avx2_sdot32(size_t n, const float *x, const float *y);        /* cpu_gemv_amd64.s:190 */
float trq_avx2_quant_dot(int dt, const float *x, const uint8_t *w, size_t K); /* cpu_quant_amd64.s */
/* quantGemv (cpu_quant.go:151-160) over the AVX2 kernels, parallel over rows. */
void trq_avx2_quant_gemv(int dt, size_t N, size_t K, const float *x, const uint8_t *w, float *c,
                         int threads);
/* quantGemvQ8/quantGemmQ8 (cpu_quant_q8.go:159-259) over AVX2 integer block kernels. */
void trq_avx2_quant_gemm_act(int dt, size_t M, size_t N, size_t K, const float *a,
                             const uint8_t *w, float *c, int threads);

#ifdef __cplusplus
}
#endif
#endif
