"""GPU parity: libtrhip through its C-ABI against the CPU oracle on the same seeded inputs.

Bit-exact wherever the reference's arithmetic is fixed: dequantization (tensor/quant.go:139-205),
the fp32 GEMV (quantDot = dequant + sdot32), the M>1 chunk order (quantGemmPanels), quantizeQ8 and
the act-quant block kernels (cpu_quant_q8.go Go twins). Shapes follow the reference's own tests
(cpu_quant_test.go, cpu_quant_q8_test.go, gpu/behavior_quant_test.go) plus the Llama-3-8B shapes.
"""
import functools

import numpy as np
import pytest

import oracle as O
from conftest import rel_err, same_bits
from tcb_amd import BLOCK, MODE_EXACT, MODE_FAST, Q4, Q4K, Q6K, Q8, TrhipError
from tcb_amd._lib import KNOB_ACTQ_TM, KNOB_EXACT_LANES, KNOB_KL
from tcb_amd import synth

pytestmark = pytest.mark.gpu

DTS = [Q8, Q4, Q4K, Q6K]
ACT_DTS = [Q4, Q4K, Q6K]


def _rng(seed):
    return np.random.default_rng(seed)


def _x(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float32)


def _weights(dt, N, K, seed):
    return O.small_scale_quant(dt, seed, N * K // BLOCK[dt][0])


@pytest.mark.parametrize("dt", DTS)
def test_store_round_trip(backend, dt):
    """ToRaw gives the uploaded GGUF bytes back (the repack is a byte permutation)."""
    N, K = 37, 2 * BLOCK[dt][0] * 4
    raw = O.random_quant(dt, 99, N * K // BLOCK[dt][0])
    w = backend.FromQuantized(dt, raw, N, K)
    assert np.array_equal(w.ToRaw(), raw)
    rb = raw.size // N
    assert np.array_equal(w.ToRaw(5, 11), raw[5 * rb:16 * rb])
    w.release()


@pytest.mark.parametrize("dt", DTS)
def test_store_chunked_upload(backend, dt):
    """A store larger than one 32 MiB upload slot (several chunks, a ragged last one) from pageable and from pinned
    host memory: ToRaw gives the GGUF bytes back and OpenQuant equals the oracle's dequantization."""
    elems, size = BLOCK[dt]
    K = 4096
    N = (70 << 20) // (K // elems * size) + 3
    raw = O.random_quant(dt, 7, N * K // elems)
    w = backend.FromQuantized(dt, raw, N, K)
    assert np.array_equal(w.ToRaw(), raw)
    h, p = backend.ctx.host_alloc(raw.nbytes)
    h[:] = raw
    w2 = backend.FromQuantized(dt, h, N, K)
    backend.ctx.host_free(p)
    assert np.array_equal(w2.ToRaw(N - 5, 5), raw[-5 * (K // elems) * size:])
    rows = 300
    out = backend.ctx.alloc(rows * K * 4)
    backend.OpenQuant(out, w2, offset=(N - rows) * K, n=rows * K)
    same_bits(out.download(np.float32, rows * K), O.dequant(dt, raw[-rows * (K // elems) * size:]))
    out.free()
    w.release()
    w2.release()


@pytest.mark.parametrize("dt", DTS)
def test_zero_store(backend, dt):
    """NewQuantStorage (tensor/quant.go:408-427): the GGUF bytes are QuantZeroRaw's (q4 codes 0x88) and OpenQuant and
    a GEMV over them give the oracle's bits. Every element is zero: +0 for q8, q4 and q4_k; q6_k opens to -0, as the
    reference's own dequantQ6K computes it (d * sc * (0 - 32) = +0 * -32, tensor/quant.go:197)."""
    elems, _ = BLOCK[dt]
    N, K = 33, 4 * elems * 2
    zero = O.quant_zero_raw(dt, N * K)
    w = backend.NewQuantStorage(dt, N, K)
    assert np.array_equal(w.ToRaw(), zero)
    out = backend.ctx.alloc(N * K * 4)
    backend.OpenQuant(out, w)
    y = out.download(np.float32, N * K)
    same_bits(y, O.dequant(dt, zero))
    assert not np.any(y)
    if dt != Q6K:
        assert not y.view(np.uint32).any()  # +0 bits
    x = synth.activations(1, K, seed=1)
    xb, cb = backend.ctx.to_device(x), backend.ctx.to_device(np.ones(N, np.float32))
    backend.GemmSet(1, N, K, xb, w, cb)
    same_bits(cb.download(np.float32, N), O.quant_gemm(dt, 1, N, K, x, zero).reshape(-1))
    for b in (out, xb, cb):
        b.free()
    w.release()


def test_memset_kernel(backend):
    """trhip_memset_async is a fill kernel: any offset and length, bytes outside the range untouched."""
    buf = backend.ctx.to_device(np.full(4096, 0x11, np.uint8))
    for off, n, v in ((0, 4096, 0), (3, 1000, 0xAB), (17, 1, 0x5C), (64, 2048, 0xFF)):
        want = buf.download(np.uint8, 4096).copy()
        want[off:off + n] = v
        backend.ctx.sync()
        from tcb_amd import _lib
        assert _lib.lib().trhip_memset_async(backend.ctx.h, buf.addr(off), v, n) == 0
        assert np.array_equal(buf.download(np.uint8, 4096), want)
    buf.free()


@pytest.mark.parametrize("dt,seed,want,at,sample", [
    (Q8, 1, 0x9994d70c2568f054, 33, 0x3a0c6000),
    (Q4K, 2, 0x9aea8c1a1a939707, 300, 0xc8f6bd40),
    (Q6K, 3, 0xf982bdb0f96cd2fc, 300, 0xc02c0000),
    (Q4, 4, 0xbe538ba4bf9b8554, 49, 0x3f328000),
])
def test_open_quant_golden(backend, dt, seed, want, at, sample):
    """OpenQuant on the card reproduces the reference's llama.cpp golden hashes (quant_test.go:55-86)."""
    elems = BLOCK[dt][0]
    raw = O.random_quant(dt, seed, 512)
    w = backend.FromQuantized(dt, raw, 512, elems)
    out = backend.ctx.alloc(512 * elems * 4)
    backend.OpenQuant(out, w)
    y = out.download(np.float32, 512 * elems)
    assert O.fnv(y) == want
    assert y.view(np.uint32)[at] == sample
    # block-aligned sub-range
    out2 = backend.ctx.alloc(3 * elems * 4)
    backend.OpenQuant(out2, w, offset=7 * elems, n=3 * elems)
    same_bits(out2.download(np.float32, 3 * elems), y[7 * elems:10 * elems])
    # an output that is not 16-byte aligned (one float into the buffer)
    out3 = backend.ctx.alloc(3 * elems * 4 + 4)
    backend.OpenQuant((out3, 4), w, offset=7 * elems, n=3 * elems)
    same_bits(out3.download(np.float32, 3 * elems, byte_offset=4), y[7 * elems:10 * elems])
    for b in (out, out2, out3):
        b.free()
    w.release()


def _gemv_case(backend, dt, N, K, seed, accumulate=True, row0=0, rows=None, x_off=0, scale=1.0):
    rng = _rng(seed)
    raw = _weights(dt, N, K, seed)
    w = backend.FromQuantized(dt, raw, N, K)
    rows = N - row0 if rows is None else rows
    x = _x(rng, K, scale)
    c0 = _x(rng, rows)
    xb = backend.ctx.alloc(K * 4 + 64)
    xb.upload(x, byte_offset=x_off)
    cb = backend.ctx.to_device(c0)
    if accumulate:
        backend.Gemm(1, rows, K, (xb, x_off), w, cb, row0=row0)
    else:
        backend.GemmSet(1, rows, K, (xb, x_off), w, cb, row0=row0)
    got = cb.download(np.float32, rows)
    rb = raw.size // N
    want = O.quant_gemm(dt, 1, rows, K, x, raw[row0 * rb:(row0 + rows) * rb], c0 if accumulate else None)
    for b in (xb, cb):
        b.free()
    w.release()
    return got, want.reshape(-1)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("N,Kb", [(1, 1), (7, 1), (9, 3), (16, 5), (33, 11), (130, 16)])
def test_gemv_exact_bits(backend, dt, N, Kb):
    """M == 1, fp32 activations: bit-identical to quantDot (TestQuantGemvMatchesOpened shapes)."""
    got, want = _gemv_case(backend, dt, N, Kb * BLOCK[dt][0], seed=N * 31 + Kb)
    same_bits(got, want)


@pytest.mark.parametrize("dt", DTS)
def test_gemv_exact_large_inputs(backend, dt):
    """x scaled by 1000 (TestQ8KernelsMatchGo's x1000 trials) stays bit-identical."""
    got, want = _gemv_case(backend, dt, 64, 2560 if dt in (Q8, Q4) else 2560, seed=5, scale=1000.0)
    same_bits(got, want)


@pytest.mark.parametrize("dt", DTS)
def test_gemv_set_slice_unaligned(backend, dt):
    """GemmSet overwrites; a row slice reads its own rows; an unaligned x is copied first."""
    K = 4 * BLOCK[dt][0]
    got, want = _gemv_case(backend, dt, 50, K, seed=7, accumulate=False)
    same_bits(got, want)
    got, want = _gemv_case(backend, dt, 50, K, seed=8, row0=10, rows=20)
    same_bits(got, want)
    got, want = _gemv_case(backend, dt, 50, K, seed=9, x_off=4)
    same_bits(got, want)


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("lanes", [4, 8, 16])
@pytest.mark.parametrize("N,Kb", [(5, 7), (33, 25), (300, 40), (2100, 9), (4096, 3)])
def test_gemv_exact_lanes_bits(backend, launch_shape, dt, lanes, N, Kb):
    """Every lane count of the exact GEMV (4, 8 or 16 lanes per row, each lane owning 8, 4 or 2 of the 32 sdot32
    chains; 16 lanes in workgroups of 4, 8 or 16 rows, with the one-wave register budget up to 4096 rows for the
    k-quants) on block counts that leave
    0 .. ring-depth - 1 blocks after the last full pass of the ring, x1 and x1000: bit-identical to quantDot."""
    launch_shape(KNOB_EXACT_LANES, lanes)
    got, want = _gemv_case(backend, dt, N, Kb * BLOCK[dt][0], seed=N + Kb + lanes, scale=1000.0 if N == 33 else 1.0)
    same_bits(got, want)


LLAMA_LINEARS = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]  # q/o, k/v, gate/up, down


@pytest.mark.parametrize("dt,N,K", [(Q4K, n, k) for n, k in LLAMA_LINEARS] + [(Q6K, n, k) for n, k in LLAMA_LINEARS] +
                         [(Q8, 4096, 4096), (Q4, 14336, 4096), (Q4, 4096, 14336)])
def test_gemv_llama_shapes_bits(backend, dt, N, K):
    """Llama-3-8B shapes with encoded N(0, 0.02) weights (1% outliers for K-quants): bit-identical."""
    raw = synth.quant_weights(dt, N, K, seed=11, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    x = synth.activations(1, K, seed=12)
    w = backend.FromQuantized(dt, raw, N, K)
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
    backend.GemmSet(1, N, K, xb, w, cb)
    got = cb.download(np.float32, N)
    want = O.quant_gemm(dt, 1, N, K, x, raw).reshape(-1)
    same_bits(got, want)
    for b in (xb, cb):
        b.free()
    w.release()


def test_gemv_empty_sum(backend):
    """K == 0: c unchanged for Gemm, zeroed for GemmSet (TestQuantGemvEdges)."""
    w = backend.FromQuantized(Q8, np.zeros(0, np.uint8), 3, 0)
    c = backend.ctx.to_device(np.array([1, 2, 3], np.float32))
    xb = backend.ctx.alloc(16)
    backend.Gemm(1, 3, 0, xb, w, c)
    assert list(c.download(np.float32, 3)) == [1, 2, 3]
    backend.GemmSet(1, 3, 0, xb, w, c)
    assert list(c.download(np.float32, 3)) == [0, 0, 0]


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("M,N,K", [(2, 40, 256), (3, 70, 512), (9, 33, 1024), (17, 20, 2560)])
def test_gemm_rows_bits(backend, dt, M, N, K):
    """M > 1, fp32 activations: bit-identical to quantGemmPanels' 256-chunk order (TestQuantMatMulSameBitsAsOpened)."""
    rng = _rng(M * 7 + N)
    raw = _weights(dt, N, K, N + K)
    w = backend.FromQuantized(dt, raw, N, K)
    x = _x(rng, M * K)
    c0 = _x(rng, M * N)
    xb, cb = backend.ctx.to_device(x), backend.ctx.to_device(c0)
    backend.Gemm(M, N, K, xb, w, cb)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm(dt, M, N, K, x, raw, c0))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q8, Q4])
@pytest.mark.parametrize("M,N,K", [(3, 50, 800), (16, 70, 2336), (7, 10300, 288)])
def test_gemm_rows_short_chunk_bits(backend, dt, M, N, K):
    """q8_0 / q4_0 rows whose last 256-wide chunk holds fewer than 8 blocks (K = 800, 2336, 288), with the chunks of
    a row block split over workgroups (few rows) and not (10300 rows)."""
    rng = _rng(M * 11 + K)
    raw = _weights(dt, N, K, N + K)
    w = backend.FromQuantized(dt, raw, N, K)
    x = _x(rng, M * K)
    c0 = _x(rng, M * N)
    xb, cb = backend.ctx.to_device(x), backend.ctx.to_device(c0)
    backend.Gemm(M, N, K, xb, w, cb)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm(dt, M, N, K, x, raw, c0))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("M,x_off,row0", [(33, 4, 0), (16, 8, 64), (5, 12, 3)])
def test_gemm_rows_unaligned_slice_bits(backend, dt, M, x_off, row0):
    """M > 1 with x at an offset that is not 16-byte aligned, a row slice of the store, and M past one pass of 16
    activation rows; x holds infinities, a NaN, zeros and subnormals."""
    N, K = 150, 512
    rng = _rng(M + x_off)
    raw = _weights(dt, N, K, M + row0)
    w = backend.FromQuantized(dt, raw, N, K)
    rows = N - row0 - 7
    x = _x(rng, M * K)
    tiny = np.array([1, 0x80000003], np.uint32).view(np.float32)
    x[3], x[K + 1], x[2 * K + 5], x[4 * K + 9:4 * K + 11] = np.inf, -np.inf, np.nan, tiny
    x[(M - 1) * K:(M - 1) * K + 64] = 0.0
    c0 = _x(rng, M * rows)
    xb = backend.ctx.alloc(M * K * 4 + 64)
    xb.upload(x, byte_offset=x_off)
    cb = backend.ctx.to_device(c0)
    backend.Gemm(M, rows, K, (xb, x_off), w, cb, row0=row0)
    rb = raw.size // N
    want = O.quant_gemm(dt, M, rows, K, x, raw[row0 * rb:(row0 + rows) * rb], c0)
    same_bits(cb.download(np.float32, M * rows), want)
    for b in (xb, cb):
        b.free()
    w.release()


def _edge_rows(K, blk):
    tiny = np.array([0x00400000], np.uint32).view(np.float32)[0]
    rows = []
    rows.append(np.zeros(K, np.float32))  # zero block
    r = np.full(K, 3.0, np.float32)
    r[1::2] = -3.0
    rows.append(r)  # saturating +-127
    r = np.full(K, 1e-3, np.float32)
    r[5] = 1000.0
    rows.append(r)  # single large
    r = np.zeros(K, np.float32)
    r[0], r[1], r[2] = tiny, -tiny / 2, tiny / 4
    rows.append(r)  # 127/amax overflows
    r = np.full(K, 0.5, np.float32)
    r[0] = 1.0
    rows.append(r)  # RNE tie 63.5 -> 64
    return np.stack(rows)


@pytest.mark.parametrize("blk", [32, 256])
def test_quantize_q8_bits(backend, blk):
    """Device quantizeQ8 == cpu_quant_q8.go:39-68 bit for bit (random rows and the edge blocks)."""
    K = 1024
    rng = _rng(blk)
    X = np.concatenate([_edge_rows(K, blk), (rng.standard_normal((6, K)) * np.array([1, 1000, 1e-30, 1, 7, 1e20])[:, None]).astype(np.float32)])
    M = X.shape[0]
    xb = backend.ctx.to_device(X)
    qb, db, bb = backend.ctx.alloc(M * K), backend.ctx.alloc(M * K // blk * 4), backend.ctx.alloc(M * K // 16 * 2)
    backend.QuantizeQ8(xb, M, K, blk, qb, db, bb)
    q = qb.download(np.int8, M * K).reshape(M, K)
    d = db.download(np.float32, M * K // blk).reshape(M, -1)
    bs = bb.download(np.int16, M * K // 16).reshape(M, -1)
    for m in range(M):
        wq, wd, wbs = O.quantize_q8(X[m], blk)
        assert np.array_equal(q[m], wq), m
        same_bits(d[m], wd)
        assert np.array_equal(bs[m], wbs), m
    for b in (xb, qb, db, bb):
        b.free()


@pytest.mark.parametrize("dt", ACT_DTS)
@pytest.mark.parametrize("M,N,K", [(1, 70, 512), (5, 7, 256), (9, 40, 2560), (13, 5, 9728), (4, 33, 512)])
def test_actq_bits(backend, dt, M, N, K):
    """GemmActQuant == quantGemmAct bit for bit (TestQ8FourRowsMatchOneRow / TestQ8EightRowsMatchOneRow shapes,
    including x1000 rows, zero-block rows and +-1 rows)."""
    rng = _rng(M * 131 + N * K)
    raw = _weights(dt, N, K, 7 * M + N + K)
    X = _x(rng, M * K).reshape(M, K)
    for m in range(M):
        if m % 5 == 1:
            X[m] *= 1000
        elif m % 5 == 2:
            X[m, :BLOCK[dt][0]] = 0
        elif m % 5 == 3:
            X[m] = 1 - 2 * (np.arange(K) % 2)
    w = backend.FromQuantized(dt, raw, N, K)
    c0 = _x(rng, M * N)
    xb, cb = backend.ctx.to_device(X), backend.ctx.to_device(c0)
    backend.GemmActQuant(M, N, K, xb, w, cb)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(dt, M, N, K, X, raw, c0))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", ACT_DTS)
@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_actq_keeps_non_finite(backend, dt, bad):
    """A row with NaN/Inf takes the fp32 path on its own; its neighbours are untouched (TestQ8PathKeepsNonFinite)."""
    M, N, K = 5, 9, 512
    rng = _rng(34)
    raw = _weights(dt, N, K, M + N)
    X = _x(rng, M * K).reshape(M, K)
    X[2, K // 2] = bad
    w = backend.FromQuantized(dt, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False)
    got = cb.download(np.float32, M * N).reshape(M, N)
    same_bits(got, O.quant_gemm_act(dt, M, N, K, X, raw))
    same_bits(got[2], O.quant_gemm(dt, 1, N, K, X[2], raw))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("M,N,K,row0,acc", [(8, 64, 256, 0, True), (130, 70, 512, 0, False), (257, 33, 1024, 5, True),
                                            (16, 200, 4096, 0, True), (128, 128, 256, 64, False), (300, 1, 512, 0, True)])
def test_actq_tiles_bits(backend, M, N, K, row0, acc):
    """Row counts that fill, straddle and overhang the 128 x 64 tiles of the MFMA prefill kernel, ragged N, a row
    slice of the store, both accumulate modes, x1000 / zero / +-1 rows and one NaN row inside a tile."""
    rng = _rng(M * 7 + N * 3 + K + row0)
    raw = _weights(Q4K, row0 + N, K, M + N + K)
    X = _x(rng, M * K).reshape(M, K)
    for m in range(M):
        if m % 7 == 1:
            X[m] *= 1000
        elif m % 7 == 2:
            X[m, :256] = 0
        elif m % 7 == 3:
            X[m] = 1 - 2 * (np.arange(K) % 2)
    if M > 20:
        X[M // 2, 3] = np.nan
    w = backend.FromQuantized(Q4K, raw, row0 + N, K)
    c0 = _x(rng, M * N) if acc else np.zeros(M * N, np.float32)
    xb, cb = backend.ctx.to_device(X), backend.ctx.to_device(c0)
    backend.GemmActQuant(M, N, K, xb, w, cb, row0=row0, accumulate=acc)
    rows = raw.reshape(row0 + N, -1)[row0:]
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(Q4K, M, N, K, X, np.ascontiguousarray(rows), c0))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("M,N,K,row0,acc", [(8, 16, 256, 0, True), (130, 70, 512, 0, False), (257, 129, 1024, 5, True),
                                            (16, 200, 4096, 0, True), (128, 128, 256, 64, False), (300, 1, 512, 0, True),
                                            (64, 1000, 2048, 3, False), (130, 16500, 256, 3, True)])
def test_actq_q6k_tiles_bits(backend, M, N, K, row0, acc):
    """q6_k act-quant on the int8 matrix cores (128 weight rows x 64 or, from 256 workgroups up, 128 activation
    rows; sub-block sums through zero-masked 16x16x64 products): row counts that fill, straddle and overhang the
    tiles, ragged N, a row slice of the store, both
    accumulate modes, x1000 / zero / +-1 rows and one NaN row inside a tile, on TR's random-scale blocks (signed
    sub-block scales of every magnitude): bit-identical to quantGemmAct."""
    rng = _rng(M * 5 + N * 3 + K + row0)
    raw = _weights(Q6K, row0 + N, K, M + N + K + 1)
    X = _x(rng, M * K).reshape(M, K)
    for m in range(M):
        if m % 7 == 1:
            X[m] *= 1000
        elif m % 7 == 2:
            X[m, :256] = 0
        elif m % 7 == 3:
            X[m] = 1 - 2 * (np.arange(K) % 2)
    if M > 20:
        X[M // 2, 3] = np.nan
    w = backend.FromQuantized(Q6K, raw, row0 + N, K)
    c0 = _x(rng, M * N) if acc else np.zeros(M * N, np.float32)
    xb, cb = backend.ctx.to_device(X), backend.ctx.to_device(c0)
    backend.GemmActQuant(M, N, K, xb, w, cb, row0=row0, accumulate=acc)
    rows = np.ascontiguousarray(raw.reshape(row0 + N, -1)[row0:])
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(Q6K, M, N, K, X, rows, c0))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("M,N,K,row0,acc", [(8, 16, 256, 0, True), (130, 70, 512, 0, False), (257, 129, 1024, 5, True),
                                            (16, 200, 4096, 0, True), (64, 128, 256, 64, False), (300, 1, 512, 0, True),
                                            (65, 1000, 2560, 3, False)])
def test_actq_q4_0_tiles_bits(backend, M, N, K, row0, acc):
    """q4_0 act-quant on the int8 matrix cores (one 32-element block per 32x32x32 product, 64 x 128 tiles, eight
    blocks per LDS stage): row counts that fill, straddle and overhang the tiles, ragged N, a row slice of the store,
    both accumulate modes, x1000 / zero / +-1 rows and one NaN row inside a tile, on TR's random-scale blocks:
    bit-identical to quantGemmAct."""
    rng = _rng(M * 7 + N * 5 + K + row0)
    raw = _weights(Q4, row0 + N, K, M + N + K + 2)
    X = _x(rng, M * K).reshape(M, K)
    for m in range(M):
        if m % 7 == 1:
            X[m] *= 1000
        elif m % 7 == 2:
            X[m, :256] = 0
        elif m % 7 == 3:
            X[m] = 1 - 2 * (np.arange(K) % 2)
    if M > 20:
        X[M // 2, 3] = np.nan
    w = backend.FromQuantized(Q4, raw, row0 + N, K)
    c0 = _x(rng, M * N) if acc else np.zeros(M * N, np.float32)
    xb, cb = backend.ctx.to_device(X), backend.ctx.to_device(c0)
    backend.GemmActQuant(M, N, K, xb, w, cb, row0=row0, accumulate=acc)
    rows = np.ascontiguousarray(raw.reshape(row0 + N, -1)[row0:])
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(Q4, M, N, K, X, rows, c0))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("weights", ["moderate", "any_scale"])
def test_actq_q4_0_scale_products_bits(backend, weights):
    """q4_0 act-quant where the per-block scale product t = fl(d_w d8) (taken on the matrix cores as a rank-1 fp32
    product) is subnormal or special: activation rows scaled from 1e-28 down to 1e-39 (d8 and t reaching the fp32
    subnormal range) and one all-zero row, on moderate weight scales and on random fp16 scale bits (subnormal and
    signed-zero d_w; NaN/Inf scales are refused when the store is made): bit-identical to quantGemmAct."""
    M, N, K = 64, 256, 1024
    rng = _rng(4400 + len(weights))
    raw = (_weights(Q4, N, K, 45) if weights == "moderate" else O.random_quant(Q4, 46, N * K // 32))
    if weights == "any_scale":  # d_w = +-0 and the smallest and largest fp16 subnormals in a few blocks
        blk = raw.reshape(N, K // 32, 18)
        for (n, b), bits in zip([(3, 5), (7, 0), (11, 31), (13, 2), (17, 9)], [0x8000, 0x0000, 0x0001, 0x83FF, 0x8001]):
            blk[n, b, 0], blk[n, b, 1] = bits & 0xFF, bits >> 8
    X = _x(rng, M * K).reshape(M, K)
    for m in range(M):
        X[m] *= np.float32(10.0 ** -(28 + m % 12)) if m % 4 else np.float32(1.0)
    X[8] = 0
    w = backend.FromQuantized(Q4, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False)
    want = O.quant_gemm_act(Q4, M, N, K, X, raw)
    assert np.count_nonzero((np.abs(want) < np.float32(1.17549435e-38)) & (want != 0)) > 0
    same_bits(cb.download(np.float32, M * N), want)
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q4, Q6K])
@pytest.mark.parametrize("N,K,M", [(14336, 4096, 512), (4096, 14336, 128)])
def test_actq_prefill_other_dtypes_bits(backend, dt, N, K, M):
    """q4_0 and q6_k act-quant at prefill sizes on encoded model weights, every output compared: bit-identical."""
    raw = synth.quant_weights(dt, N, K, seed=43, outliers=0.01 if dt == Q6K else 0.0)
    X = synth.activations(M, K, seed=44 + M)
    w = backend.FromQuantized(dt, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(dt, M, N, K, X, raw))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q4K, Q6K])
@pytest.mark.parametrize("M,N,K,row0,acc,x_off", [(300, 16421, 512, 5, True, 0), (257, 49153, 256, 0, False, 4),
                                                  (384, 12800, 1024, 0, True, 0), (260, 16640, 768, 9, False, 0)])
def test_prefill_tiles_bits(backend, dt, M, N, K, row0, acc, x_off):
    """The 128-row-per-wave prefill kernels, q4_k and q6_k (taken for grids of at least 192 128x256 tiles; 384 x
    12800 is below that and takes the other kernels): rows padded past M, ragged N, a row slice of the store, both
    accumulate modes, an unaligned x, x1000 / zero / +-1 rows and a NaN row (its outputs from the fp32 path), on TR's
    random-scale blocks (q6_k: signed sub-block scales of every magnitude): bit-identical to the oracle."""
    rng = _rng(M + N + K)
    raw = _weights(dt, row0 + N, K, M * 3 + K)
    X = _x(rng, M * K).reshape(M, K)
    X[1] *= 1000
    X[2, :256] = 0
    X[3] = 1 - 2 * (np.arange(K) % 2)
    X[M - 2, 11] = np.nan
    w = backend.FromQuantized(dt, raw, row0 + N, K)
    c0 = _x(rng, M * N) if acc else np.zeros(M * N, np.float32)
    xb = backend.ctx.alloc(M * K * 4 + 16)
    xb.upload(X, byte_offset=x_off)
    cb = backend.ctx.to_device(c0)
    backend.GemmActQuant(M, N, K, (xb, x_off), w, cb, row0=row0, accumulate=acc)
    rows = np.ascontiguousarray(raw.reshape(row0 + N, -1)[row0:])
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(dt, M, N, K, X, rows, c0))
    for b in (xb, cb):
        b.free()
    w.release()


def test_prefill_q6k_extreme_bits(backend):
    """q6_k prefill at the ends of the plane split: codes 0 and 63 under sub-block scales -128, -1, 0, 1 and 127 (the
    products (q - 32) sc reach 4096, -4064 and 3937), against activations at the code limits +-127 (constant rows,
    alternating rows) and ordinary rows: bit-identical to the oracle."""
    M, N, K = 256, 24576, 512
    rng = _rng(7)
    nb = K // 256
    blk = np.zeros((N, nb, 210), np.uint8)
    code = rng.integers(0, 2, size=(N, nb)) * 63  # all codes 0 or all 63 per block
    blk[:, :, 0:128] = np.where(code[..., None] == 63, 0xFF, 0x00)
    blk[:, :, 128:192] = np.where(code[..., None] == 63, 0xFF, 0x00)
    scales = np.array([-128, -1, 0, 1, 127], np.int8).view(np.uint8)
    blk[:, :, 192:208] = scales[rng.integers(0, 5, size=(N, nb, 16))]
    blk[:, :, 208:210] = np.array([0x00, 0x3C], np.uint8)  # d = 1.0
    raw = blk.reshape(-1)
    X = _x(rng, M * K).reshape(M, K)
    X[0] = 3.0
    X[1] = -3.0
    X[2] = np.where(np.arange(K) % 2 == 0, 5.0, -5.0)
    X[3, ::256] = 100.0
    w = backend.FromQuantized(Q6K, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(Q6K, M, N, K, X, raw))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt,N,K,M", [(Q4, 14336, 4096, 8), (Q4, 4096, 14336, 8), (Q4K, 4096, 4096, 16),
                                      (Q6K, 1024, 4096, 16)])
def test_gemm_rows_llama_shapes_bits(backend, dt, N, K, M):
    """Decode batches on Llama shapes through the fp32 M>1 path: q4_0 FFN at batch 8, q4_k / q6_k at batch 16."""
    raw = synth.quant_weights(dt, N, K, seed=31, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    X = synth.activations(M, K, seed=32)
    w = backend.FromQuantized(dt, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmSet(M, N, K, xb, w, cb)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm(dt, M, N, K, X, raw))
    for b in (xb, cb):
        b.free()
    w.release()


@functools.lru_cache(maxsize=2)
def _ffn_q4k(N, K):
    return synth.quant_weights(Q4K, N, K, seed=41, outliers=0.01)


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("M", [128, 512, 2048])
def test_actq_prefill_sizes_bits(backend, N, K, M):
    """The prefill configurations (q4_k, M in {128, 512, 2048}), every output row and column compared: each is one
    single-row kernel result (cpu_quant_q8.go:183-185), bit-identical."""
    raw = _ffn_q4k(N, K)
    X = synth.activations(M, K, seed=42 + M)
    w = backend.FromQuantized(Q4K, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False)
    got = cb.download(np.float32, M * N).reshape(M, N)
    same_bits(got, O.quant_gemm_act(Q4K, M, N, K, X, raw))
    for b in (xb, cb):
        b.free()
    w.release()


def _q4k_weights_f64(raw, N, K):
    """q4_k weights d (sc q) - dmin m in float64 without the fp32 roundings of the dequant: sc q and m are recovered
    exactly as the dequant of the same blocks with (d, dmin) set to (1, 0) and (0, 1), and d, dmin read from the
    blocks' fp16 fields."""
    blk = np.array(raw, np.uint8).reshape(-1, 144)
    one, zero = np.array([0x00, 0x3C], np.uint8), np.array([0, 0], np.uint8)  # fp16 1.0 and +0
    a, b = blk.copy(), blk.copy()
    a[:, 0:2], a[:, 2:4] = one, zero
    b[:, 0:2], b[:, 2:4] = zero, one
    scq = O.dequant(Q4K, a.reshape(-1)).astype(np.float64).reshape(-1, 256)
    negm = O.dequant(Q4K, b.reshape(-1)).astype(np.float64).reshape(-1, 256)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64)
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float64)
    return (d * scq + dmin * negm).reshape(N, K)


def _run_actq_modes(backend, raw, X, M, N, K, row0, c0, acc):
    """Fast twice and exact once on the same inputs; returns the three outputs as [M, N]."""
    w = backend.FromQuantized(Q4K, raw, row0 + N, K)
    xb = backend.ctx.to_device(X)
    outs = []
    for md in (MODE_FAST, MODE_FAST, MODE_EXACT):
        cb = backend.ctx.to_device(c0)
        backend.GemmActQuant(M, N, K, xb, w, cb, row0=row0, accumulate=acc, mode=md)
        outs.append(cb.download(np.float32, M * N).reshape(M, N))
        cb.free()
    xb.free()
    w.release()
    return outs


@pytest.mark.parametrize("M,N,K,row0,acc", [(8, 64, 256, 0, True), (130, 70, 512, 0, False), (300, 16421, 512, 5, True),
                                            (384, 12800, 1024, 0, False), (128, 14336, 4096, 0, False),
                                            (512, 14336, 4096, 0, False), (512, 4096, 14336, 0, True),
                                            (128, 4096, 14336, 0, True), (2048, 4096, 14336, 0, False)])
def test_actq_fast_within_tolerance(backend, M, N, K, row0, acc):
    """Fast act-quant (trhip_gemm_q_actq_mode) on encoded model weights: the same quantized activations and exact
    integer block sums with the fp32 epilogue fused, on both matrix-core kernels (64-row tiles below, 128 rows
    per wave from 192 128x256 tiles up): within the K-quant bound 1e-4 of quantGemmAct by |a-b|/(1+|b|), the same
    bits on every call, NaN rows as the exact path computes them (fp32 fallback), and different bits from the exact
    mode somewhere (the fused kernel ran). The x1000 row is compared at its input's scale (both results divided by
    1000), as the fast GEMV tests compare theirs: its outputs are 1000 times larger, so an output that cancels to
    a small value carries rounding at the 1000-fold scale in either order."""
    rng = _rng(M + N + K + 7)
    raw = _ffn_q4k(N, K) if (N, K) in ((14336, 4096), (4096, 14336)) and row0 == 0 else \
        synth.quant_weights(Q4K, row0 + N, K, seed=M + K, outliers=0.01)
    X = _x(rng, M * K).reshape(M, K)
    X[1] *= 1000
    X[2, :256] = 0
    X[M - 2, 11] = np.nan
    c0 = _x(rng, M * N) if acc else np.zeros(M * N, np.float32)
    fast, fast2, exact = _run_actq_modes(backend, raw, X, M, N, K, row0, c0, acc)
    same_bits(fast, fast2)
    rows = np.ascontiguousarray(raw.reshape(row0 + N, -1)[row0:])
    want = O.quant_gemm_act(Q4K, M, N, K, X, rows, c0).reshape(M, N)
    same_bits(exact, want)
    same_bits(fast[M - 2], want[M - 2])
    fin = np.ones(M, bool)
    fin[M - 2] = False
    fin[1] = False
    assert rel_err(fast[fin], want[fin]) <= 1e-4
    assert rel_err(fast[1] / np.float32(1000), want[1] / np.float32(1000)) <= 1e-4
    assert not np.array_equal(fast[fin].view(np.uint32), want[fin].view(np.uint32))


@pytest.mark.parametrize("M,N,K", [(64, 300, 1024), (384, 12800, 1024), (512, 2048, 4096), (128, 300, 14336)])
def test_actq_fast_random_scale_blocks(backend, M, N, K):
    """Fast act-quant on TR's random-scale blocks (cpu_quant_test.go:71-86), whose rows cancel: d isum and
    dmin msum nearly cancel inside each block, so any fp32 rounding order of the epilogue lands ulps of the large
    terms apart. Held to the standard of the fast GEMV on these blocks: against the float64 value of the same
    quantized product (q8 codes times their scales, times the dequantized weights: the value both epilogues round),
    the fast result is no further than 1e-4 or twice the exact path's own distance, whichever is larger."""
    rng = _rng(M * 3 + K)
    raw = _weights(Q4K, N, K, N + K + M)
    X = _x(rng, M * K).reshape(M, K)
    c0 = np.zeros(M * N, np.float32)
    fast, fast2, exact = _run_actq_modes(backend, raw, X, M, N, K, 0, c0, False)
    same_bits(fast, fast2)
    same_bits(exact, O.quant_gemm_act(Q4K, M, N, K, X, raw))
    q, d8, _ = O.quantize_q8(X, 256)
    xq = (q.astype(np.float64).reshape(M, K // 256, 256) * d8.astype(np.float64).reshape(M, K // 256, 1)).reshape(M, K)
    truth = xq @ _q4k_weights_f64(raw, N, K).T
    fast_err, exact_err = rel_err(fast, truth), rel_err(exact, truth)
    assert fast_err <= max(1e-4, 2.0 * exact_err), (M, N, K, fast_err, exact_err)


@pytest.mark.parametrize("S", [2, 3, 8])
@pytest.mark.parametrize("tm", [32, 64])
def test_actq_fast_k_slices(backend, launch_shape, tm, S):
    """Fast act-quant with K cut into S slices (the last workgroup of a tile adds the partials in slice order):
    within 1e-4 of quantGemmAct on model weights on ragged tiles with a row slice and accumulation, the same bits
    on every call, the x1000 row at its input's scale and the NaN row as the exact path computes it."""
    M, N, K, row0 = 96, 700, 8192, 3
    launch_shape(KNOB_ACTQ_TM, tm, S)
    rng = _rng(S + tm)
    raw = synth.quant_weights(Q4K, row0 + N, K, seed=S + 11, outliers=0.01)
    X = _x(rng, M * K).reshape(M, K)
    X[1] *= 1000
    X[M - 2, 5000] = np.nan
    c0 = _x(rng, M * N)
    fast, fast2, exact = _run_actq_modes(backend, raw, X, M, N, K, row0, c0, True)
    same_bits(fast, fast2)
    rows = np.ascontiguousarray(raw.reshape(row0 + N, -1)[row0:])
    want = O.quant_gemm_act(Q4K, M, N, K, X, rows, c0).reshape(M, N)
    same_bits(exact, want)
    same_bits(fast[M - 2], want[M - 2])
    fin = np.ones(M, bool)
    fin[[1, M - 2]] = False
    assert rel_err(fast[fin], want[fin]) <= 1e-4
    assert rel_err(fast[1] / np.float32(1000), want[1] / np.float32(1000)) <= 1e-4


@pytest.mark.parametrize("dt", [Q4, Q6K])
def test_actq_fast_other_dtypes_exact(backend, dt):
    """q4_0 and q6_k act-quant have no fused epilogue: fast mode gives the exact bits."""
    M, N, K = 16, 300, 2048
    raw = _weights(dt, N, K, 5)
    X = _x(_rng(9), M * K).reshape(M, K)
    w = backend.FromQuantized(dt, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False, mode=MODE_FAST)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(dt, M, N, K, X, raw))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("M", [97, 128])
def test_gemm_rows_above_panel_bits(backend, dt, M):
    """M > 96 takes the reference's other M > 1 driver (cpu_quant.go:59-82, quantGemm without panels); it keeps the
    256-deep chunk order per output, so the result is the same bits as below 96 rows (TestQuantMatMulSameBitsAsOpened
    at a larger M)."""
    N, K = 300, 4096
    raw = synth.quant_weights(dt, N, K, seed=61 + M, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    X = synth.activations(M, K, seed=62)
    X[5] *= 1000
    w = backend.FromQuantized(dt, raw, N, K)
    c0 = synth.activations(M, N, seed=63).reshape(-1)
    xb, cb = backend.ctx.to_device(X), backend.ctx.to_device(c0)
    backend.Gemm(M, N, K, xb, w, cb)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm(dt, M, N, K, X, raw, c0))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q4K, Q6K])
def test_gemv_k16384(backend, dt):
    """K = 16384, the largest K the fast M == 1 kernels take (four K parts of 16 blocks): exact bit-identical, fast
    within the bound."""
    N, K = 500, 16384
    raw = synth.quant_weights(dt, N, K, seed=71, outliers=0.01)
    x = synth.activations(1, K, seed=72)
    w = backend.FromQuantized(dt, raw, N, K)
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
    want = O.quant_gemm(dt, 1, N, K, x, raw).reshape(-1)
    backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_EXACT)
    same_bits(cb.download(np.float32, N), want)
    backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
    assert rel_err(cb.download(np.float32, N), want) <= FAST_TOL[dt]
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt,N,K,M", [(Q4K, 14336, 4096, 16), (Q4K, 4096, 14336, 8), (Q6K, 1024, 4096, 32),
                                      (Q4, 4096, 4096, 16)])
def test_actq_llama_shapes_bits(backend, dt, N, K, M):
    raw = synth.quant_weights(dt, N, K, seed=21, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    X = synth.activations(M, K, seed=22)
    w = backend.FromQuantized(dt, raw, N, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm_act(dt, M, N, K, X, raw))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", DTS)
def test_embedding(backend, dt):
    """Selected rows dequantized (TestQuantEmbedding); an out-of-range row is refused (H3043)."""
    D = 512
    raw = O.random_quant(dt, 9, 5 * D // BLOCK[dt][0])
    w = backend.FromQuantized(dt, raw, 5, D)
    idx = [4, 0, 4, 2]
    out = backend.ctx.alloc(len(idx) * D * 4)
    backend.Embedding(out, w, idx)
    same_bits(out.download(np.float32, len(idx) * D), O.embedding(dt, raw, D, idx))
    out1 = backend.ctx.alloc(len(idx) * D * 4 + 4)  # an output that is not 16-byte aligned
    backend.Embedding((out1, 4), w, idx)
    same_bits(out1.download(np.float32, len(idx) * D, byte_offset=4), O.embedding(dt, raw, D, idx))
    with pytest.raises(TrhipError):
        backend.Embedding(out, w, [5])
    # back-to-back lookups with no sync between them: the pinned index staging is reused only after its copy ran
    outs = [backend.ctx.alloc(3 * D * 4) for _ in range(4)]
    picks = [[1, 2, 3], [3, 3, 0], [4, 1, 2], [0, 0, 0]]
    for o, ix in zip(outs, picks):
        backend.Embedding(o, w, ix)
    for o, ix in zip(outs, picks):
        same_bits(o.download(np.float32, 3 * D), O.embedding(dt, raw, D, ix))
    for b in [out, out1] + outs:
        b.free()
    w.release()


def test_actq_refuses_q8(backend):
    w = backend.FromQuantized(Q8, O.random_quant(Q8, 1, 2), 2, 32)
    xb, cb = backend.ctx.alloc(128), backend.ctx.alloc(8)
    with pytest.raises(TrhipError) as e:
        backend.GemmActQuant(1, 2, 32, xb, w, cb)
    assert e.value.code == 5


def test_store_refuses_bad_scale(backend):
    raw = O.random_quant(Q8, 3, 3)
    raw[34 + 1] = 0x7C  # block 1 scale -> +Inf
    with pytest.raises(TrhipError) as e:
        backend.FromQuantized(Q8, raw, 3, 32)
    assert e.value.code == 7


# ---------------------------------------------------------------- fast mode (tolerance-bound)
FAST_TOL = {Q8: 1e-5, Q4: 1e-5, Q4K: 1e-4, Q6K: 1e-4}  # fast-mode bound: 1e-5, 1e-4 for K-quants


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("N,K", [(7, 256), (64, 512), (130, 2048), (33, 4096), (200, 14336), (1024, 4096),
                                 (14336, 4096), (4096, 14336)])
def test_gemv_fast_tolerance(backend, dt, N, K):
    """MODE_FAST: |gpu - oracle| / (1 + |oracle|) within the fast-mode bound, for accumulate and set,
    on encoded N(0, 0.02) weights with 1% outliers and on x1000 activations."""
    raw = synth.quant_weights(dt, N, K, seed=N + K, outliers=0.01)
    w = backend.FromQuantized(dt, raw, N, K)
    for scale, acc in ((1.0, False), (1000.0, True)):
        x = synth.activations(1, K, seed=K) * np.float32(scale)
        c0 = synth.activations(1, N, seed=N).reshape(-1)
        xb, cb = backend.ctx.to_device(x), backend.ctx.to_device(c0)
        if acc:
            backend.Gemm(1, N, K, xb, w, cb, mode=MODE_FAST)
        else:
            backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
        got = cb.download(np.float32, N)
        want = O.quant_gemm(dt, 1, N, K, x, raw, c0 if acc else None).reshape(-1)
        err = rel_err(got / scale, want / scale)
        assert err <= FAST_TOL[dt], (dt, N, K, scale, err)
        for b in (xb, cb):
            b.free()
    w.release()


@pytest.mark.parametrize("N,K", LLAMA_LINEARS + [(6144, 4096), (7000, 4096), (28672, 4096)])
def test_gemv_fast_llama_shapes(backend, N, K):
    """The fast q4_k GEMV on every Llama-3-8B linear shape and the merged [q | k | v] (6144) and [gate | up] (28672)
    stores, plus a ragged 7000 rows (encoded weights with 1% outliers), within 1e-4."""
    raw = synth.quant_weights(Q4K, N, K, seed=51, outliers=0.01)
    x = synth.activations(1, K, seed=52)
    w = backend.FromQuantized(Q4K, raw, N, K)
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
    backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
    err = rel_err(cb.download(np.float32, N), O.quant_gemm(Q4K, 1, N, K, x, raw).reshape(-1))
    assert err <= FAST_TOL[Q4K], err
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", DTS)
def test_gemv_fast_deterministic_and_sliced(backend, dt):
    """Same input, same bits on every call (no atomic accumulation; TestQuantGemvIsDeterministic), and a
    row slice computes the slice's rows."""
    N, K = 300, 14336 if dt in (Q4K, Q6K) else 4096
    raw = synth.quant_weights(dt, N, K, seed=5, outliers=0.01)
    w = backend.FromQuantized(dt, raw, N, K)
    x = synth.activations(1, K, seed=6)
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
    backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
    first = cb.download(np.float32, N)
    for _ in range(3):
        backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
        same_bits(cb.download(np.float32, N), first)
    backend.GemmSet(1, 100, K, xb, w, cb, row0=123, mode=MODE_FAST)
    same_bits(cb.download(np.float32, 100), first[123:223])
    for b in (xb, cb):
        b.free()
    w.release()


# q4_k fast GEMV with K across lanes (fixed-point x, int8 dot products); the launch_shape fixture forces a shape
KL_SHAPES = ["4,1,4,8", "4,1,4,16", "4,1,2,16", "8,1,4,8", "4,2,4,16", "8,4,4,8"]


def _kl_parts(cfg):
    return int(cfg.split(",")[1])


@pytest.mark.parametrize("cfg", KL_SHAPES)
@pytest.mark.parametrize("N,K,row0", [(1, 256, 0), (37, 1024, 0), (300, 4096, 5), (129, 3840, 0), (9000, 4096, 100),
                                      (70, 14336, 3), (40, 8192, 0)])
def test_gemv_kl_tolerance(backend, launch_shape, cfg, N, K, row0):
    """Every launch shape of the K-across-lanes kernel on ragged shapes (rows fewer than row groups, partial K
    parts, a row slice), set and accumulate, x1 and x1000 activations: within 1e-4 of the oracle. Shapes whose
    K needs more than 16 blocks per part are refused."""
    launch_shape(KNOB_KL, *map(int, cfg.split(",")))
    rows = N
    raw = synth.quant_weights(Q4K, N + row0, K, seed=N + K, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N + row0, K)
    if -(-(K // 256) // _kl_parts(cfg)) > 16:
        xb, cb = backend.ctx.alloc(K * 4), backend.ctx.alloc(rows * 4)
        with pytest.raises(TrhipError) as e:
            backend.GemmSet(1, rows, K, xb, w, cb, row0=row0, mode=MODE_FAST)
        assert e.value.code == 5
        for b in (xb, cb):
            b.free()
        w.release()
        return
    sub = raw.reshape(N + row0, -1)[row0:].reshape(-1)
    for scale, acc in ((1.0, False), (1000.0, True)):
        x = synth.activations(1, K, seed=K + 1) * np.float32(scale)
        c0 = synth.activations(1, rows, seed=rows).reshape(-1)
        xb, cb = backend.ctx.to_device(x), backend.ctx.to_device(c0)
        if acc:
            backend.Gemm(1, rows, K, xb, w, cb, row0=row0, mode=MODE_FAST)
        else:
            backend.GemmSet(1, rows, K, xb, w, cb, row0=row0, mode=MODE_FAST)
        want = O.quant_gemm(Q4K, 1, rows, K, x, sub, c0 if acc else None).reshape(-1)
        err = rel_err(cb.download(np.float32, rows) / scale, want / scale)
        assert err <= FAST_TOL[Q4K], (cfg, N, K, row0, scale, err)
        for b in (xb, cb):
            b.free()
    w.release()


@pytest.mark.parametrize("cfg", ["4,1,4,16", "8,4,4,8"])
def test_gemv_kl_activation_range(backend, launch_shape, cfg):
    """Fixed-point x is scaled per 32-element half: one huge element among tiny ones, an all-zero half, subnormal
    activations and activations near 1e35 stay within tolerance (zero x gives zero rows)."""
    launch_shape(KNOB_KL, *map(int, cfg.split(",")))
    N, K = 64, 4096 if _kl_parts(cfg) == 1 else 14336
    raw = synth.quant_weights(Q4K, N, K, seed=8, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N, K)
    rng = _rng(3)
    xs = []
    x = (rng.standard_normal(K) * 1e-3).astype(np.float32)
    x[5], x[700] = 1e4, -3e3
    x[64:96] = 0
    xs.append(x)
    xs.append((rng.standard_normal(K) * 1e-40).astype(np.float32))  # subnormal
    xs.append(np.zeros(K, np.float32))
    xs.append((rng.standard_normal(K) * 1e30).astype(np.float32))
    xs.append((rng.standard_normal(K) * 1e35).astype(np.float32))  # sums far from overflow, sc * X * 2^e near it
    for x in xs:
        xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
        backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
        got = cb.download(np.float32, N)
        want = O.quant_gemm(Q4K, 1, N, K, x, raw).reshape(-1)
        amax = float(np.max(np.abs(x))) or 1.0
        if amax < 1e-30:
            # subnormal products: the oracle's own K fused steps each round to the 2^-149 grid
            assert float(np.max(np.abs(got.astype(np.float64) - want))) <= K * 2.0 ** -149
        else:
            assert rel_err(got / amax, want / amax) <= FAST_TOL[Q4K]
        if not x.any():
            assert not got.any()
        for b in (xb, cb):
            b.free()
    w.release()


@pytest.mark.parametrize("cfg", ["4,1,4,16", "8,4,4,8"])
@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_gemv_kl_non_finite(backend, launch_shape, cfg, bad):
    """Inf or NaN in x takes float products in the lanes that hold it: every row is NaN or +-Inf exactly where the
    bit-exact GEMV is (a zero weight times Inf is NaN, as on the CPU)."""
    launch_shape(KNOB_KL, *map(int, cfg.split(",")))
    N, K = 48, 4096 if _kl_parts(cfg) == 1 else 14336
    raw = synth.quant_weights(Q4K, N, K, seed=4, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N, K)
    x = synth.activations(1, K, seed=5).reshape(-1)
    x[1234] = bad
    xb, cb, eb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4), backend.ctx.alloc(N * 4)
    backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
    backend.GemmSet(1, N, K, xb, w, eb, mode=MODE_EXACT)
    got, exact = cb.download(np.float32, N), eb.download(np.float32, N)
    assert np.array_equal(np.isnan(got), np.isnan(exact))
    assert np.array_equal(np.isposinf(got), np.isposinf(exact))
    assert np.array_equal(np.isneginf(got), np.isneginf(exact))
    for b in (xb, cb, eb):
        b.free()
    w.release()


# ---------------------------------------------------------------- merged layers and the SwiGLU epilogue
def test_swiglu_bits(backend):
    """trhip_swiglu == siluForward then the product, bit for bit (layers.tr:223), on N(0, 5) values and the edge
    values of the exp kernel's clamps, overflow, subnormals, infinities, NaN and -0."""
    rng = _rng(21)
    for M, I in ((3, 1000), (2, 7), (1, 1)):
        gu = (rng.standard_normal((M, 2 * I)) * 5).astype(np.float32)
        edge = np.array([np.inf, -np.inf, np.nan, -0.0, 0.0, -200, -103.97, -87.4, 88.5, 89, 1e-40, -1e-40, 1e30, -1e30],
                        np.float32)
        flat = gu.reshape(-1)
        flat[:min(edge.size, flat.size)] = edge[:min(edge.size, flat.size)]
        flat[-min(edge.size, flat.size):] = edge[:min(edge.size, flat.size)]
        gb, ob = backend.ctx.to_device(gu), backend.ctx.alloc(M * I * 4)
        backend.SwiGLU(gb, M, I, ob)
        same_bits(ob.download(np.float32, M * I), O.swiglu(gu, M, I).reshape(-1))
        for b in (gb, ob):
            b.free()


@pytest.mark.parametrize("dt", DTS)
def test_wstore_concat(backend, dt):
    """A merged store holds the parts' rows in order: ToRaw gives the concatenated bytes, and every GEMV / act-quant
    GEMM on it equals the parts' results side by side (exact modes bit for bit)."""
    K = 2 * BLOCK[dt][0] * 4
    Ns = (37, 5, 64)
    raws = [_weights(dt, n, K, 40 + i) for i, n in enumerate(Ns)]
    parts = [backend.FromQuantized(dt, r, n, K) for r, n in zip(raws, Ns)]
    w = parts[0].Concat(parts)
    N = sum(Ns)
    assert w.N == N
    assert np.array_equal(w.ToRaw(), np.concatenate(raws))
    rng = _rng(5)
    for M in (1, 3):
        x = _x(rng, M * K).reshape(M, K)
        xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(M * N * 4)
        backend.GemmSet(M, N, K, xb, w, cb)
        want = np.concatenate([O.quant_gemm(dt, M, n, K, x, r) for r, n in zip(raws, Ns)], axis=1)
        same_bits(cb.download(np.float32, M * N), want.reshape(-1))
        if dt != Q8:
            backend.GemmActQuant(M, N, K, xb, w, cb, accumulate=False)
            want = np.concatenate([O.quant_gemm_act(dt, M, n, K, x, r) for r, n in zip(raws, Ns)], axis=1)
            same_bits(cb.download(np.float32, M * N), want.reshape(-1))
        for b in (xb, cb):
            b.free()
    other = backend.FromQuantized(dt, _weights(dt, 3, 2 * K, 9), 3, 2 * K)
    with pytest.raises(TrhipError) as e:
        parts[0].Concat([parts[0], other])
    assert e.value.code == 1
    for p in parts + [w, other]:
        p.release()


@pytest.mark.parametrize("dt", [Q4K, Q6K, Q4])
@pytest.mark.parametrize("M", [1, 3, 16])
def test_gemm_q_swiglu_bits(backend, dt, M):
    """SwiGLU.forward's gate/up half on a merged [gate | up] store: exact mode is the reference's matmul followed by
    swiglu_gate, bit for bit. Fast mode: the merged GEMV is within the dtype's tolerance of the exact one, and the
    fused result is swiglu_gate of that fast GEMV bit for bit (the tolerance bounds the GEMV; silu(g) * u scales
    g's absolute error by |u|, so it is not a bound on the product)."""
    I, K = 300, 1024
    graw, uraw = _weights(dt, I, K, 11), _weights(dt, I, K, 12)
    wg, wu = backend.FromQuantized(dt, graw, I, K), backend.FromQuantized(dt, uraw, I, K)
    w = wg.Concat([wg, wu])
    rng = _rng(M)
    x = _x(rng, M * K).reshape(M, K)
    xb, ob = backend.ctx.to_device(x), backend.ctx.alloc(M * I * 4)
    backend.GemmSwiGLU(M, K, xb, w, ob)
    gu = np.concatenate([O.quant_gemm(dt, M, I, K, x, graw), O.quant_gemm(dt, M, I, K, x, uraw)], axis=1)
    want = O.swiglu(gu, M, I).reshape(-1)
    same_bits(ob.download(np.float32, M * I), want)
    # fast mode (M > 1 on matrix cores: the gate fused into the K-slice sum)
    gub = backend.ctx.alloc(M * 2 * I * 4)
    backend.GemmSet(M, 2 * I, K, xb, w, gub, mode=MODE_FAST)
    gu_fast = gub.download(np.float32, M * 2 * I)
    assert rel_err(gu_fast, gu.reshape(-1)) <= FAST_TOL[dt]
    backend.GemmSwiGLU(M, K, xb, w, ob, mode=MODE_FAST)
    same_bits(ob.download(np.float32, M * I), O.swiglu(gu_fast.reshape(M, 2 * I), M, I).reshape(-1))
    gub.free()
    odd = backend.FromQuantized(dt, _weights(dt, 3, K, 1), 3, K)
    with pytest.raises(TrhipError):
        backend.GemmSwiGLU(M, K, xb, odd, ob)
    for b in (xb, ob):
        b.free()
    for p in (wg, wu, w, odd):
        p.release()


@pytest.mark.parametrize("dt", [Q4K, Q6K])
@pytest.mark.parametrize("M,I,K", [(16, 300, 256), (16, 1000, 4096), (8, 700, 2048)])
def test_gemm_q_swiglu_fast_rows(backend, dt, M, I, K):
    """Fast M > 1: the gate fused into the K-slice sum (or applied after the kernel when K is one slice) gives
    the bits of the fast GEMM followed by swiglu_gate."""
    raw = synth.quant_weights(dt, 2 * I, K, seed=I + M, outliers=0.01)
    w = backend.FromQuantized(dt, raw, 2 * I, K)
    X = synth.activations(M, K, seed=K + M)
    xb, gub, ob = backend.ctx.to_device(X), backend.ctx.alloc(M * 2 * I * 4), backend.ctx.alloc(M * I * 4)
    backend.GemmSet(M, 2 * I, K, xb, w, gub, mode=MODE_FAST)
    gu = gub.download(np.float32, M * 2 * I).reshape(M, 2 * I)
    backend.GemmSwiGLU(M, K, xb, w, ob, mode=MODE_FAST)
    same_bits(ob.download(np.float32, M * I), O.swiglu(gu, M, I).reshape(-1))
    for b in (xb, gub, ob):
        b.free()
    w.release()


@pytest.mark.parametrize("I,K", [(3100, 4096), (5120, 4096), (14336, 4096), (3100, 2048)])
def test_gemm_q_swiglu_fused_fast(backend, I, K):
    """Fast decode with the SwiGLU gate fused into the q4_k GEMV (merged [gate | up] stores of 6144 or more rows):
    the same bits as the fast GEMV over the merged store followed by swiglu_gate, for an aligned and an unaligned x
    (the latter takes the two-step path); the GEMV within the q4_k bound of the exact one."""
    raw = synth.quant_weights(Q4K, 2 * I, K, seed=I + K, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, 2 * I, K)
    x = synth.activations(1, K, seed=K + 1)
    xb = backend.ctx.alloc(K * 4 + 64)
    gub, ob = backend.ctx.alloc(2 * I * 4), backend.ctx.alloc(I * 4)
    for off in (0, 4):
        xb.upload(x, byte_offset=off)
        backend.GemmSet(1, 2 * I, K, (xb, off), w, gub, mode=MODE_FAST)
        gu = gub.download(np.float32, 2 * I)
        backend.GemmSwiGLU(1, K, (xb, off), w, ob, mode=MODE_FAST)
        same_bits(ob.download(np.float32, I), O.swiglu(gu.reshape(1, 2 * I), 1, I).reshape(-1))
    want = O.quant_gemm(Q4K, 1, 2 * I, K, x, raw).reshape(-1)
    assert rel_err(gu, want) <= FAST_TOL[Q4K]
    for b in (xb, gub, ob):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("M", [1, 3, 16])
@pytest.mark.parametrize("N,K", [(300, 1024), (6144, 4096), (700, 14336), (10240, 2048)])
def test_fast_random_scale_blocks(backend, dt, M, N, K):
    """Every fast kernel (the M = 1 GEMVs, both q4_k layouts, and the M > 1 matrix-core paths) on TR's random
    blocks with moderate random scales (cpu_quant_test.go:71-86), x ~ N(0, 1).

    Such rows cancel: sum |w x| is 10^3 to 10^5 times |y|, so the exact fp32 sum is itself 1e-5 to 5e-4 away
    from the float64 value of the same product, and no other summation order can stay within 1e-5 of its
    rounding. Two bounds are checked: the reference's own GPU-against-CPU rule for these blocks,
    |a - b| / (1 + |b|) <= 1e-5 sqrt(K) (gpu/behavior_quant_test.go:298, :395); and against the float64 product,
    the fast result is no further than the dtype's bound or twice the exact path's own distance, whichever is
    larger. (The fixed-point grid error, about rms(w) 2^-23 max|x| sqrt(K), is the same order as the fp32
    rounding of the exact sum here; the measured ratio of the two distances is 0.4 to 1.05.)"""
    raw = _weights(dt, N, K, N + K + M)
    w = backend.FromQuantized(dt, raw, N, K)
    X = _x(_rng(M + K), M * K).reshape(M, K)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmSet(M, N, K, xb, w, cb, mode=MODE_FAST)
    got = cb.download(np.float32, M * N)
    exact = O.quant_gemm(dt, M, N, K, X, raw).reshape(-1)
    err = rel_err(got, exact)
    assert err <= 1e-5 * np.sqrt(K), (dt, M, N, K, err)
    truth = (X.astype(np.float64) @ O.dequant(dt, raw).reshape(N, K).astype(np.float64).T).reshape(-1)
    fast_err, exact_err = rel_err(got, truth), rel_err(exact, truth)
    assert fast_err <= max(FAST_TOL[dt], 2.0 * exact_err), (dt, M, N, K, fast_err, exact_err)
    for b in (xb, cb):
        b.free()
    w.release()


FASTM_SHAPES = [(5, 100, 256, 0), (8, 300, 4096, 5), (16, 1000, 4096, 0), (17, 129, 3840, 3), (33, 70, 14336, 0),
                (64, 9000, 4096, 0)]


@pytest.mark.parametrize("dt", [Q4K, Q6K])
@pytest.mark.parametrize("M,N,K,row0", FASTM_SHAPES)
def test_gemm_rows_fast_tolerance(backend, dt, M, N, K, row0):
    """Fast-mode M > 1 (int8 matrix cores over fixed-point activations): within the dtype's bound of the oracle on
    ragged shapes, row slices, set and accumulate, x1 and x1000 activations, an unaligned x; two calls agree bit
    for bit."""
    raw = synth.quant_weights(dt, N + row0, K, seed=N + K, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    w = backend.FromQuantized(dt, raw, N + row0, K)
    sub = raw.reshape(N + row0, -1)[row0:].reshape(-1)
    for scale, acc, off in ((1.0, False, 0), (1000.0, True, 4)):
        x = synth.activations(M, K, seed=K + M) * np.float32(scale)
        c0 = synth.activations(M, N, seed=N).reshape(-1)
        xb = backend.ctx.alloc(M * K * 4 + 64)
        xb.upload(x, byte_offset=off)
        outs = []
        for _ in range(2):
            cb = backend.ctx.to_device(c0)
            if acc:
                backend.Gemm(M, N, K, (xb, off), w, cb, row0=row0, mode=MODE_FAST)
            else:
                backend.GemmSet(M, N, K, (xb, off), w, cb, row0=row0, mode=MODE_FAST)
            outs.append(cb.download(np.float32, M * N))
            cb.free()
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        want = O.quant_gemm(dt, M, N, K, x, sub, c0 if acc else None).reshape(-1)
        err = rel_err(outs[0] / scale, want / scale)
        assert err <= FAST_TOL[dt], (dt, M, N, K, row0, scale, err)
        xb.free()
    w.release()


@pytest.mark.parametrize("dt", [Q4K, Q6K])
def test_gemm_rows_fast_activation_range(backend, dt):
    """Each 256-wide block of each activation row has its own fixed-point exponent: one huge element among tiny
    ones, an all-zero block, subnormal rows, 1e30 rows and zero rows in one call stay within tolerance."""
    N, K = 200, 4096
    raw = synth.quant_weights(dt, N, K, seed=8, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    w = backend.FromQuantized(dt, raw, N, K)
    rng = _rng(3)
    X = np.zeros((6, K), np.float32)
    X[0] = rng.standard_normal(K) * 1e-3
    X[0, 5], X[0, 700] = 1e4, -3e3
    X[0, 256:512] = 0
    X[1] = rng.standard_normal(K) * 1e-40  # subnormal
    X[3] = rng.standard_normal(K) * 1e30
    X[4] = rng.standard_normal(K)
    X[5, :256] = rng.standard_normal(256) * 1e-20
    X[5, 256:] = rng.standard_normal(K - 256) * 1e20
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(6 * N * 4)
    backend.GemmSet(6, N, K, xb, w, cb, mode=MODE_FAST)
    got = cb.download(np.float32, 6 * N).reshape(6, N)
    want = O.quant_gemm(dt, 6, N, K, X, raw).reshape(6, N)
    for m in range(6):
        amax = float(np.max(np.abs(X[m]))) or 1.0
        if amax < 1e-30:
            assert float(np.max(np.abs(got[m].astype(np.float64) - want[m]))) <= K * 2.0 ** -149
        else:
            assert rel_err(got[m] / amax, want[m] / amax) <= FAST_TOL[dt], m
    assert not got[2].any()
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q4K, Q6K])
@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_gemm_rows_fast_non_finite(backend, dt, bad):
    """Rows of x holding Inf or NaN are computed with float products: NaN / +-Inf exactly where the exact path has
    them, the other rows within tolerance."""
    M, N, K = 5, 150, 4096
    raw = synth.quant_weights(dt, N, K, seed=4, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    w = backend.FromQuantized(dt, raw, N, K)
    X = synth.activations(M, K, seed=6)
    X[1, 777] = bad
    X[3, 4095] = bad
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmSet(M, N, K, xb, w, cb, mode=MODE_FAST)
    got = cb.download(np.float32, M * N).reshape(M, N)
    want = O.quant_gemm(dt, M, N, K, X, raw).reshape(M, N)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    assert np.array_equal(np.sign(got[~fin & ~np.isnan(want)]), np.sign(want[~fin & ~np.isnan(want)]))
    assert rel_err(got[fin], want[fin]) <= FAST_TOL[dt]
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q8, Q4])
def test_gemm_rows_fast_other_dtypes_exact(backend, dt):
    """At M > 1 the fast mode of q8_0, and of q4_0 where K is not a multiple of 256 (rows16.hip takes q4_0 at
    2..16 rows in 256-element chunks), is the exact path: the same bits as mode exact."""
    M, N = 6, 70
    for K in ((512, 32 * 9) if dt == Q8 else (32 * 9,)):
        raw = _weights(dt, N, K, 5)
        w = backend.FromQuantized(dt, raw, N, K)
        x = _x(_rng(2), M * K)
        xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(M * N * 4)
        backend.GemmSet(M, N, K, xb, w, cb, mode=MODE_FAST)
        same_bits(cb.download(np.float32, M * N), O.quant_gemm(dt, M, N, K, x, raw))
        for b in (xb, cb):
            b.free()
        w.release()


def test_gemm_rows_fast_small_m_exact(backend):
    """Fast mode with q4_k and M <= 4 runs the exact kernel: the same bits as mode exact."""
    M, N, K = 4, 90, 1024
    raw = _weights(Q4K, N, K, 6)
    w = backend.FromQuantized(Q4K, raw, N, K)
    x = _x(_rng(8), M * K)
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(M * N * 4)
    backend.GemmSet(M, N, K, xb, w, cb, mode=MODE_FAST)
    same_bits(cb.download(np.float32, M * N), O.quant_gemm(Q4K, M, N, K, x, raw))
    for b in (xb, cb):
        b.free()
    w.release()


Q84_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (300, 1024), (77, 8192)]


@pytest.mark.parametrize("dt", [Q8, Q4, Q6K])
@pytest.mark.parametrize("N,K", Q84_SHAPES)
def test_gemv_fast_q8_q4(backend, dt, N, K):
    """Fast q8_0 / q4_0 / q6_k GEMV (K across lanes over fixed-point x) on the Llama-3-8B shapes and ragged ones,
    set and accumulate, x1 and x1000: within the 1e-5 (q8_0, q4_0) and 1e-4 (q6_k) bounds."""
    raw = synth.quant_weights(dt, N, K, seed=N + 3 * K, outliers=0.01 if dt == Q6K else 0.0)
    w = backend.FromQuantized(dt, raw, N, K)
    for scale, acc in ((1.0, False), (1000.0, True)):
        x = synth.activations(1, K, seed=K + 7) * np.float32(scale)
        c0 = synth.activations(1, N, seed=N + 1).reshape(-1)
        xb, cb = backend.ctx.to_device(x), backend.ctx.to_device(c0)
        if acc:
            backend.Gemm(1, N, K, xb, w, cb, mode=MODE_FAST)
        else:
            backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
        want = O.quant_gemm(dt, 1, N, K, x, raw, c0 if acc else None).reshape(-1)
        err = rel_err(cb.download(np.float32, N) / scale, want / scale)
        assert err <= FAST_TOL[dt], (dt, N, K, scale, err)
        for b in (xb, cb):
            b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q8, Q4, Q6K])
@pytest.mark.parametrize("cfg", ["4,1,4,8", "4,1,4,16", "4,1,2,16", "8,1,4,8", "4,2,4,16", "4,2,4,8", "8,2,4,8",
                                 "8,4,4,8"])
def test_gemv_fast_q8_q4_launch_shapes(backend, launch_shape, dt, cfg):
    """Every launch shape of the K-across-lanes kernel for q8_0 / q4_0 / q6_k on ragged rows and K parts (K = 8192
    and 2560: parts of up to 128 blocks of 32, or 16 of 256), within the bound; shapes whose parts exceed that are
    refused."""
    launch_shape(KNOB_KL, *map(int, cfg.split(",")))
    ks = int(cfg.split(",")[1])
    for N, K in ((133, 8192), (70, 2560)):
        raw = synth.quant_weights(dt, N, K, seed=N + K, outliers=0.01 if dt == Q6K else 0.0)
        w = backend.FromQuantized(dt, raw, N, K)
        x = synth.activations(1, K, seed=K)
        xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
        nb = K // BLOCK[dt][0]
        too_big = (nb + ks - 1) // ks > 16 if dt == Q6K else ((nb + ks - 1) // ks + 1) // 2 * 2 > 128
        if too_big:
            with pytest.raises(TrhipError) as e:
                backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
            assert e.value.code == 5
        else:
            backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
            err = rel_err(cb.download(np.float32, N), O.quant_gemm(dt, 1, N, K, x, raw).reshape(-1))
            assert err <= FAST_TOL[dt], (cfg, N, K, err)
        for b in (xb, cb):
            b.free()
        w.release()


@pytest.mark.parametrize("dt", [Q8, Q4, Q6K])
@pytest.mark.parametrize("bad", [np.inf, np.nan])
def test_gemv_fast_q8_q4_non_finite(backend, dt, bad):
    """Inf / NaN in x: float products in the lanes that hold it, NaN and +-Inf exactly where the exact GEMV has
    them."""
    N, K = 90, 4096
    raw = synth.quant_weights(dt, N, K, seed=12)
    w = backend.FromQuantized(dt, raw, N, K)
    x = synth.activations(1, K, seed=13).reshape(-1)
    x[1000] = bad
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
    backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
    got = cb.download(np.float32, N)
    want = O.quant_gemm(dt, 1, N, K, x, raw).reshape(-1)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    assert np.array_equal(np.sign(got[~fin & ~np.isnan(want)]), np.sign(want[~fin & ~np.isnan(want)]))
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("dt", [Q8, Q4])
def test_gemv_fast_q8_q4_odd_blocks_exact(backend, dt):
    """An odd number of 32-element blocks per row does not fit two blocks per lane: the fast mode runs the exact
    kernel (same bits as mode exact)."""
    N, K = 50, 32 * 9
    raw = _weights(dt, N, K, 3)
    w = backend.FromQuantized(dt, raw, N, K)
    x = _x(_rng(4), K)
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(N * 4)
    backend.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
    same_bits(cb.download(np.float32, N), O.quant_gemm(dt, 1, N, K, x, raw).reshape(-1))
    for b in (xb, cb):
        b.free()
    w.release()


def test_read_probe(backend):
    """The streaming-read diagnostic reads an aligned buffer and writes nothing; unaligned sizes are refused."""
    buf = backend.ctx.to_device(np.arange(4096, dtype=np.float32))
    backend.ctx.read_probe(buf)
    backend.ctx.read_probe(buf, 0)
    backend.ctx.sync()
    assert np.array_equal(buf.download(np.float32, 4096), np.arange(4096, dtype=np.float32))
    with pytest.raises(TrhipError) as e:
        backend.ctx.read_probe(buf, 100)
    assert e.value.code == 1
    buf.free()


def test_mfma_probe(backend):
    """The int8 matrix-core diagnostic runs for every VALU mix it has and refuses others."""
    from tcb_amd import _lib
    L = _lib.lib()
    for v in (0, 2, 4, 6, 8, 12, 16):
        assert L.trhip_mfma_probe(backend.ctx.h, v, 2, 8) == 0
    assert L.trhip_mfma_probe(backend.ctx.h, 5, 2, 8) == 1
    assert L.trhip_mfma_probe(backend.ctx.h, 0, 5, 8) == 1
    backend.ctx.sync()


def test_prefill_probe_runs_and_refuses(backend):
    """trhip_prefill_probe runs the three inner loops on a prefill grid and refuses bad kinds and shapes."""
    from tcb_amd import _lib
    L = _lib.lib()
    h = backend.ctx.h
    for kind in (0, 1, 2):
        assert L.trhip_prefill_probe(h, kind, 512, 14336, 4096) == 0
    backend.ctx.sync()
    assert L.trhip_prefill_probe(h, 3, 512, 14336, 4096) == 1
    assert L.trhip_prefill_probe(h, 1, 512, 14336, 4000) == 1
    assert L.trhip_prefill_probe(h, 1, 0, 14336, 4096) == 1
    backend.ctx.sync()
