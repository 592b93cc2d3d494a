/*
 * trhip.h -- C-ABI of libtrhip, the MI355X (gfx950) implementation of TR's quantized GGUF
 * matmul. Plain integers and pointers only, so the Go runtime can bind it through purego
 * or cgo. Reference citations are relative to the reference repository root; "tensor/"
 * means internal/compute/tensor/ and "gpu/" means internal/compute/gpu/.
 *
 * Conventions
 *  - Every entry point returns an int status (TRHIP_OK == 0). Nothing aborts and nothing
 *    throws across the ABI. trhip_last_error(ctx) gives the detail text of the last
 *    failure on that context; trhip_strerror(code) names a code.
 *  - A context owns one device and one in-order HIP stream. Calls on one context must be
 *    serialized by the caller (the reference takes one backend lock per call,
 *    gpu/gpu.go:211-232). Work is asynchronous until trhip_sync / trhip_d2h.
 *  - Weights are [N, K] quantized rows (blocks along K), activations x are fp32 [M, K]
 *    row-major, outputs c are fp32 [M, N] row-major (f16 or bf16 either side through
 *    trhip_gemm_q_typed); x and c are device pointers from trhip_alloc (or any device
 *    allocation on the context's device).
 */
#ifndef TRHIP_H
#define TRHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The reference reports coded panics (messages.New(H...)); out-of-memory is
 * a catchable error there too (docs/spec/15_tensorler.md:528). */
enum {
    TRHIP_OK = 0,
    TRHIP_ERR_INVALID = 1,     /* bad argument / shape / dtype                          */
    TRHIP_ERR_OOM = 2,         /* device allocation failed                              */
    TRHIP_ERR_HIP = 3,         /* HIP runtime error (name in trhip_last_error)          */
    TRHIP_ERR_LAUNCH = 4,      /* kernel launch failed                                  */
    TRHIP_ERR_UNSUPPORTED = 5, /* dtype not supported by this operator (e.g. act-quant q8) */
    TRHIP_ERR_NO_DEVICE = 6,   /* no HIP device / driver                                */
    TRHIP_ERR_BAD_SCALE = 7    /* NaN/Inf fp16 scale (H6686)                             */
};

/* Quantized dtypes; same block formats as tensor/quant.go:23-47 and gguf/types.go:31-41. */
enum { TRHIP_Q8 = 1, TRHIP_Q4 = 2, TRHIP_Q4K = 3, TRHIP_Q6K = 4 };

/* GEMV arithmetic for fp32 activations (trhip_gemm_q with M == 1).
 * EXACT: bit-identical to TR's CPU quantDot (dequant + sdot32 order).
 * FAST:  per-sub-block factored sums; within 1e-5 (q8_0, q4_0) or 1e-4 (q4_k, q6_k) of EXACT by
 *        |a - b| / (1 + |b|), not bit-identical. */
enum { TRHIP_MODE_EXACT = 0, TRHIP_MODE_FAST = 1 };

/* Element types of activations and outputs for trhip_gemm_q_typed (fp32 everywhere else). */
enum { TRHIP_F32 = 0, TRHIP_F16 = 1, TRHIP_BF16 = 2 };

typedef struct trhip_ctx trhip_ctx;
typedef struct trhip_wstore trhip_wstore;

const char *trhip_strerror(int code);
const char *trhip_last_error(const trhip_ctx *ctx);
int trhip_version(void);

/* Replaces the lazy GPU backend set-up: tensor/device_registry.go:51 (RegisterLazyBackend),
 * gpu/gpu.go:86-170 (Count, setupFn). */
int trhip_device_count(int *count);
int trhip_init(int device, trhip_ctx **out);
/* Destroy order: every weight store and graph made on ctx first, then ctx. While any is alive,
 * trhip_destroy returns TRHIP_ERR_INVALID and leaves the context (and them) working. */
int trhip_destroy(trhip_ctx *ctx);
/* The context's stream as a hipStream_t (for callers that interleave their own work). */
void *trhip_stream(trhip_ctx *ctx);

/* Device memory; replaces Backend.Alloc and the loadHost/download pair
 * (tensor/device.go:393, gpu/memory.go:524). */
int trhip_alloc(trhip_ctx *ctx, size_t bytes, void **dptr);
int trhip_free(trhip_ctx *ctx, void *dptr);
int trhip_h2d_async(trhip_ctx *ctx, void *dst, const void *src, size_t bytes);
int trhip_d2h(trhip_ctx *ctx, void *dst, const void *src, size_t bytes); /* waits */
/* A fill kernel (not a memset node), so it may be captured into a graph like the compute calls. */
int trhip_memset_async(trhip_ctx *ctx, void *dst, int value, size_t bytes);
/* trhip_d2h, trhip_sync and trhip_free wait for the stream and fail with TRHIP_ERR_INVALID while it is captured. */
int trhip_sync(trhip_ctx *ctx);

/* Page-locked host memory (the off-heap HostBlock of tensor/host_block.go:150-200 can live here):
 * trhip_wstore_create uploads a source inside such a block by DMA from where it is, with no staging copy. */
int trhip_host_alloc(trhip_ctx *ctx, size_t bytes, void **hptr);
int trhip_host_free(trhip_ctx *ctx, void *hptr);

/* Stream-ordered timing events (the reference's TR_GPU_PROFILE events, gpu/profile.go:1-34). */
int trhip_event_create(trhip_ctx *ctx, void **ev);
int trhip_event_record(trhip_ctx *ctx, void *ev);
int trhip_event_elapsed_ms(void *ev_start, void *ev_end, float *ms);
int trhip_event_destroy(void *ev);

/* Stream capture into a replayable HIP graph (launch-bound sequences such as a decode sweep).
 * Every call made on ctx between begin and end is recorded, not run; trhip_graph_launch replays it
 * on the context's stream. Calls that would grow the context's workspace fail during capture: make
 * one eager call of the same shapes first. A graph's nodes address the workspace as it was at
 * capture; when a later eager call grows it, the old buffers stay allocated until the context's last
 * graph is destroyed, so replays stay valid. Calls that wait for the stream, allocate or free
 * (trhip_sync, trhip_d2h, trhip_free, store creation and release, host-index embedding) refuse while
 * capturing. Counterpart of the reference's CUDA-graph replay (gpu/graph.go); nothing on this path
 * requires it. */
int trhip_graph_begin(trhip_ctx *ctx);
int trhip_graph_end(trhip_ctx *ctx, void **exec);
int trhip_graph_launch(trhip_ctx *ctx, void *exec);
int trhip_graph_destroy(void *exec);

/* Load gate, tensor/quant.go:108-128 (CheckQuantScales): index of the first block with a
 * NaN/Inf fp16 scale in *bad_block, or -1. Host-side, no device needed. */
int trhip_check_quant_scales(int dtype, const void *raw, size_t raw_bytes, int64_t *bad_block);

/* Device-resident weight store. Replaces RawBackend.FromRaw for quantized dtypes
 * (tensor/typed.go:22-30, gpu/typed.go:24-35, tensor/quant.go:75-81) and the load path
 * FromHostBlock -> FromQuantized (tensor/host_block.go:180-186, stdlib/ml/load_gguf.go:79-107):
 * raw holds N*K/blk GGUF blocks in file order. They are uploaded in chunks through pinned
 * staging (a source inside a trhip_host_alloc block is sent by DMA directly) and repacked on
 * the device into per-field planes (codes, scales) for 128-bit coalesced loads. No value is
 * decoded. A pageable source is copied before the call returns; a pinned one must stay valid
 * until the next trhip_sync on ctx. The scale gate of trhip_check_quant_scales runs on the host
 * while earlier chunks are in flight; a bad block (TRHIP_ERR_BAD_SCALE, H6686) drops the store. */
int trhip_wstore_create(trhip_ctx *ctx, int dtype, const void *raw, size_t raw_bytes, int64_t N,
                        int64_t K, trhip_wstore **out);
/* Zeroed quantized storage, tensor/quant.go:408-427 (newQuantStorage / QuantZeroRaw): every block
 * byte 0 except the q4 codes, 0x88, so that every element opens to zero: +0 for q8_0, q4_0 and
 * q4_k, and -0 for q6_k (d*sc*(0-32) with d = +0), as the reference's dequantQ6K gives. */
int trhip_wstore_create_zero(trhip_ctx *ctx, int dtype, int64_t N, int64_t K, trhip_wstore **out);
int trhip_wstore_destroy(trhip_wstore *w); /* Releaser.Release, tensor/device.go:520-522 */
int trhip_wstore_info(const trhip_wstore *w, int *dtype, int64_t *N, int64_t *K, size_t *device_bytes);
/* One store holding the rows of several (same dtype and K), in order: the merged layers of
 * lib/layers.tr (gate_up_proj = [gate | up], layers.tr:240-262; merged q/k/v weights) as one
 * device store, so one GEMV reads the shared activation once. The parts stay valid. */
int trhip_wstore_concat(trhip_ctx *ctx, const trhip_wstore *const *parts, int nparts, trhip_wstore **out);
/* RawBackend.ToRaw (tensor/typed.go:27): the original GGUF bytes of rows [row0, row0+rows). */
int trhip_wstore_to_raw(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t rows, void *raw_out);

/* Backend.Gemm / GemmSet for a quantized right operand (tensor/device.go:478,
 * tensor/device_registry.go:193-195, tensor/cpu_dtype.go:448-466, gpu/backend_quant.go:43-65):
 *   c[m, n] (+)= sum_k x[m, k] * deq(w)[row0 + n, k],  m < M, n < N, k < K.
 * accumulate != 0 is Gemm (c +=), 0 is GemmSet (c =). K must equal the store's K and
 * row0 + N <= store N (row slices, tensor/quant.go:266-272). M == 1 is the decode GEMV
 * (tensor/cpu_quant.go:151); M > 1 follows quantGemmPanels' 256-deep chunk order
 * (tensor/cpu_quant.go:103-147). K == 0 is the empty sum (c unchanged, zeroed when
 * accumulate == 0). mode: TRHIP_MODE_EXACT, or TRHIP_MODE_FAST: deterministic and within 1e-4
 * (q4_k, q6_k) or 1e-5 (q8_0, q4_0) of the exact result, |a - b| / (1 + |b|). Fast mode runs the
 * M == 1 GEMV of every dtype on fixed-point activations (K up to 16384; q8_0 / q4_0 with an even
 * block count), q4_k with 5 <= M <= 16 on f16 matrix cores over two-term activations and with M > 16
 * on int8 matrix cores, q4_0 with 2 <= M <= 16 (K a multiple of 256) and q6_k with M > 1 on f16 matrix
 * cores; other cases run exact. The reference GPU's GEMV and its M > 1 dequantize-and-GEMM are tolerance-bound too
 * (gpu/kernel_quant_gemv.go:33-84, gpu/backend_quant.go:43-134). */
int trhip_gemm_q(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x,
                 float *c, int64_t M, int64_t K, int accumulate, int mode);

/* trhip_gemm_q with 16-bit activations and / or outputs (xtype, ctype: TRHIP_F32, TRHIP_F16, TRHIP_BF16; x holds
 * M*K and c M*N elements of their type), as the reference's quantGemm takes them (gpu/backend_quant.go:41-45,
 * gpu/backend_memory.go:41-52, 98-115): x is widened to fp32 exactly, the product is trhip_gemm_q's in fp32 (c
 * widened first when accumulating), and c is rounded to its type once, to nearest even (tensor/cpu_dtype.go:73-123:
 * NaN stays a quiet NaN, f16 overflows to Inf). Bit-identical to widening x, calling trhip_gemm_q and rounding its
 * result. With x and c of one 16-bit type (x 8-byte and c 2-byte aligned) the batch-1 GEMV (both modes) and the
 * fast batched decode read and write them directly; other cases go through fp32 copies in a workspace of the
 * context. */
int trhip_gemm_q_typed(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const void *x, int xtype,
                       void *c, int ctype, int64_t M, int64_t K, int accumulate, int mode);

/* ActQuantGemmer.GemmActQuant (tensor/matmul.go:59-61, tensor/cpu_dtype.go:438-446 ->
 * tensor/cpu_quant_q8.go:125-259): x rows are quantized on the device to Q8 blocks of the
 * weight's block size (quantizeQ8), integer block sums are exact int32 (int8 MFMA for M >= 8: q4_k, q6_k, and
 * q4_0 when the row's block count is a multiple of 8; packed int8 dot products otherwise), and the per-block
 * fp32 epilogue follows the reference order, so outputs are bit-identical to the CPU path.
 * Rows holding NaN/Inf use the fp32 path for that row only. dtype must be q4, q4_k or q6_k
 * (QuantActSupported, tensor/cpu_quant_q8.go:122), else TRHIP_ERR_UNSUPPORTED. */
int trhip_gemm_q_actq(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x,
                      float *c, int64_t M, int64_t K, int accumulate);

/* trhip_gemm_q_actq with a mode, as trhip_gemm_q takes one (the reference's GemmActQuant has no mode; this is
 * the same operator). TRHIP_MODE_EXACT is trhip_gemm_q_actq. TRHIP_MODE_FAST keeps the quantized activations and
 * the exact int32 block sums (isum, msum) and fuses the per-block fp32 epilogue (two fma instead of two products,
 * a difference and a sum) on the q4_k matrix-core kernels: deterministic and within 1e-4 of the exact result,
 * |a - b| / (1 + |b|); other dtypes and small M run exact. */
int trhip_gemm_q_actq_mode(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x,
                           float *c, int64_t M, int64_t K, int accumulate, int mode);

/* No counterpart in the reference: trhip_gemm_q_actq for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments, kernels and bits as
 * trhip_gemm_q_actq, but the quantized activations live in a static device array of
 * TRHIP_NOALLOC_SCRATCH_BYTES per device instead of the context's workspace, and nothing is allocated or freed.
 * Shapes whose scratch exceeds it (about 1.27 M*K bytes, plus 4 M*K when x is not 16-byte aligned; M = 2048 at
 * K = 14336 fits) fail with TRHIP_ERR_INVALID before anything runs. Every call on one device shares that array:
 * calls that overlap on one device (two contexts, or two streams) race. No part of the array needs to start at
 * zero. */
#define TRHIP_NOALLOC_SCRATCH_BYTES (40u << 20)
int trhip_gemm_q_actq_noalloc(trhip_ctx *ctx, const trhip_wstore *w, int64_t row0, int64_t N, const float *x,
                              float *c, int64_t M, int64_t K, int accumulate);

/* QuantOpener.OpenQuant (tensor/quant.go:103-105, gpu/backend_quant.go:117-134): elements
 * [elem_off, elem_off+n) of the store in row-major order, dequantized to fp32, bit-identical
 * to tensor/quant.go:139-205. elem_off and n must be multiples of the block size. */
int trhip_open_q(trhip_ctx *ctx, const trhip_wstore *w, int64_t elem_off, int64_t n, float *out);

/* Backend.Embedding for a quantized table (tensor/device.go:482, tensor/cpu_quant.go:163-171):
 * out[i, :] = deq(w)[idx[i], :]; idx is a host array of nidx int64 row indices (the reference passes
 * a Go []int). Indices are checked on the host before upload; an out-of-range index returns
 * TRHIP_ERR_INVALID (H3043). The indices are copied to pinned staging and uploaded asynchronously;
 * the caller's array may be reused on return. Refused while the stream is captured. */
int trhip_embedding_q(trhip_ctx *ctx, const trhip_wstore *w, const int64_t *idx, int64_t nidx, float *out);

/* SwiGLU gate (lib/layers.tr:223 swiglu_gate on the [gate | up] halves of a merged gate_up output,
 * layers.tr:240-262): out[m, i] = silu(gu[m, i]) * gu[m, I + i] for a [M, 2I] row-major gu, with silu as
 * tensor/cpu_elementwise_wide.go:101-116 and e^x as the AVX2 expVec (tensor/cpu_vector_amd64.s:13-38):
 * bit-identical to the CPU path. */
int trhip_swiglu(trhip_ctx *ctx, const float *gu, int64_t M, int64_t I, float *out);

/* SwiGLU.forward's first half on a merged store (lib/layers.tr:264-266): gu = x @ w^T over all 2I rows
 * ([gate | up], trhip_gemm_q semantics and mode), then out = trhip_swiglu(gu). out is [M, I]. In fast mode
 * with M == 1 the gate is fused into the q4_k GEMV where its K-across-lanes kernel applies (2I >= 6144, K a
 * multiple of 256 up to 4096, 16-byte aligned x): the same bits as the two steps. */
int trhip_gemm_q_swiglu(trhip_ctx *ctx, const trhip_wstore *w, const float *x, float *out, int64_t M,
                        int64_t K, int mode);

/* Quantize fp32 rows to Q8 activation blocks on the device (tensor/cpu_quant_q8.go:39-68):
 * q [M, K] int8, d [M, K/blk] fp32, bs [M, K/16] int16; blk is 32 or 256. Exposed for
 * parity tests and for callers that reuse one quantized activation across weights. */
int trhip_quantize_q8(trhip_ctx *ctx, const float *x, int64_t M, int64_t K, int blk, int8_t *q, float *d,
                      int16_t *bs);

/* Diagnostic with no counterpart in the reference: reads `bytes` of device memory at p once (p and
 * bytes 16-byte aligned) and writes nothing. One launch over a buffer that is not in the caches times
 * the device's single-launch streaming-read ceiling, the floor the GEMV kernels are measured against. */
int trhip_read_probe(trhip_ctx *ctx, const void *p, int64_t bytes);

/* Diagnostic with no counterpart in the reference: one workgroup per CU of 4 * waves_per_simd waves, each running
 * iters rounds of four independent v_mfma_i32_32x32x32_i8 (262,144 int8 ops per round) with valu_per_mfma
 * (0, 2, 4, 6, 8, 12 or 16) independent fp32 FMAs issued beside each MFMA. Timed with events it gives the device's
 * int8 matrix-core rate and how much VALU work hides under it, the ceiling of the prefill kernel. */
int trhip_mfma_probe(trhip_ctx *ctx, int valu_per_mfma, int waves_per_simd, int64_t iters);

/* Diagnostic with no counterpart in the reference: the act-quant prefill kernel's inner loop alone (kind 0: q4_k
 * exact, 1: q4_k fast, 2: q6_k), on the grid trhip_gemm_q_actq launches for M x N x K, with its LDS staging, its
 * per-block barrier and its stores taken out (weights and activations are not read). Timed with events it gives the
 * ceiling of the loop the prefill kernel runs per block. Refused during graph capture. */
int trhip_prefill_probe(trhip_ctx *ctx, int kind, int64_t M, int64_t N, int64_t K);

/* Test and tuning hook with no counterpart in the reference: force a launch shape on this context
 * instead of the built-in choice (all four values 0 restores it). Shapes that are not built are
 * refused here, never at a later GEMV. TRHIP_KNOB_KL: K-across-lanes fast GEMV (a, b, c, d) =
 * (waves, K parts, rows in flight, rows per wave); TRHIP_KNOB_FAST_Q4K: row-sliced fast q4_k GEMV
 * (blocks in flight, waves, K parts, rows per lane); TRHIP_KNOB_EXACT_ROWS: exact four-lane GEMV rows
 * per workgroup a; TRHIP_KNOB_EXACT_LANES: exact GEMV lanes per row a (4, 8 or 16); TRHIP_KNOB_ACTQ_TM: act-quant
 * MFMA row tile a (0: built-in) and, in fast mode, b K slices (0: built-in); TRHIP_KNOB_ROWS16: fast q4_k kernel for 2..16 activation rows (a, b) = (16-row tiles per
 * wave 1 or 2; K slices 1..64, clamped to the block count); TRHIP_KNOB_KL_GRID: at least a workgroups for
 * the K-across-lanes fast GEMV (its rows dealt over more, shorter row groups). */
enum { TRHIP_KNOB_KL = 1, TRHIP_KNOB_FAST_Q4K = 2, TRHIP_KNOB_EXACT_ROWS = 3, TRHIP_KNOB_EXACT_LANES = 4,
       TRHIP_KNOB_ACTQ_TM = 5, TRHIP_KNOB_ROWS16 = 6, TRHIP_KNOB_KL_GRID = 7 };
int trhip_set_launch_shape(trhip_ctx *ctx, int knob, int a, int b, int c, int d);

#ifdef __cplusplus
}
#endif
#endif
