"""16-bit activations and outputs through trhip_gemm_q_typed, as the reference's quantGemm takes them
(gpu/backend_quant.go:41-45, gpu/backend_memory.go:41-52, 98-115): a widened to float32 exactly, the float32 product
(c widened first when accumulating), c rounded once to nearest even (tensor/cpu_dtype.go:73-123).

Exact mode: bit-identical to the oracle's product on the widened activations, rounded by the oracle's restatement of
the reference's conversions. Fast mode: bit-identical to the fp32 fast call on the same widened activations followed
by the same rounding, both where the batch-1 GEMV reads and writes 16-bit data directly and where the call goes through
fp32 copies."""
import numpy as np
import pytest

import oracle as O
from tcb_amd import BF16, F16, F32, MODE_EXACT, MODE_FAST, Q4, Q4K, Q6K, Q8, synth

pytestmark = pytest.mark.gpu
SIZE = {F32: 4, F16: 2, BF16: 2}


def _in(t, x):
    """Activations of type t: (device bytes as a numpy array, the exact float32 values they hold)."""
    if t == F32:
        return x.astype(np.float32), x.astype(np.float32)
    h = O.round16(t, x)
    return h, O.widen16(t, h)


def _widen(t, raw):
    return raw.view(np.float32) if t == F32 else O.widen16(t, raw)


def _out(t, y):
    return y.astype(np.float32).view(np.uint32) if t == F32 else O.round16(t, y)


def _same(got, want, t):
    """Bit equality of t-typed results (NaN compared by NaN-ness)."""
    g, w = np.asarray(got).reshape(-1), np.asarray(want).reshape(-1)
    assert g.shape == w.shape
    gn, wn = np.isnan(_widen(t, g)), np.isnan(_widen(t, w))
    assert np.array_equal(gn, wn), "NaN positions differ"
    bad = np.nonzero(g[~gn] != w[~wn])[0]
    assert bad.size == 0, f"{bad.size} of {g.size} differ, first at {bad[0]}: {g[~gn][bad[0]]:#x} != {w[~wn][bad[0]]:#x}"


def _fast32(backend, w, N, K, xw, cw, acc):
    """The fp32 fast GEMV of the widened activations (on the widened c when accumulating)."""
    xb, cb = backend.ctx.to_device(xw), backend.ctx.to_device(cw)
    (backend.Gemm if acc else backend.GemmSet)(1, N, K, xb, w, cb, mode=MODE_FAST)
    y = cb.download(np.float32, N)
    xb.free()
    cb.free()
    return y


def _run(backend, w, M, N, K, xa, xt, c0, ct, acc, mode, row0=0):
    xb = backend.ctx.to_device(xa)
    cb = backend.ctx.to_device(c0)
    backend.GemmTyped(M, N, K, xb, xt, w, cb, ct, row0=row0, accumulate=acc, mode=mode)
    got = cb.download(np.uint32 if ct == F32 else np.uint16, M * N)
    xb.free()
    cb.free()
    return got


@pytest.mark.parametrize("xt,ct", [(F16, F16), (BF16, BF16), (F16, F32), (F32, BF16), (BF16, F16)])
@pytest.mark.parametrize("dt,M,N,K", [(Q4K, 1, 300, 4096), (Q6K, 3, 77, 2048), (Q8, 1, 130, 1024),
                                      (Q4, 5, 64, 2560), (Q4K, 16, 200, 1024)])
@pytest.mark.parametrize("acc", [False, True])
def test_typed_exact_bits(backend, xt, ct, dt, M, N, K, acc):
    """Exact mode: c = round(c_widened (+) oracle product of the widened activations), every combination of types."""
    raw = synth.quant_weights(dt, N, K, seed=N + K, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    w = backend.FromQuantized(dt, raw, N, K)
    rng = np.random.default_rng(M * N + K)
    xa, xw = _in(xt, (rng.standard_normal(M * K) * 3).astype(np.float32))
    ca, cw = _in(ct, (rng.standard_normal(M * N) * 5).astype(np.float32))
    got = _run(backend, w, M, N, K, xa, xt, ca, ct, acc, MODE_EXACT)
    want = O.quant_gemm(dt, M, N, K, xw.reshape(M, K), raw, cw if acc else None).reshape(-1)
    _same(got, _out(ct, want), ct)
    w.release()


@pytest.mark.parametrize("t", [F16, BF16])
@pytest.mark.parametrize("dt,N,K", [(Q4K, 14336, 4096), (Q4K, 4096, 14336), (Q4K, 1000, 2048), (Q6K, 4096, 4096),
                                    (Q6K, 1024, 14336), (Q8, 4096, 4096), (Q4, 14336, 4096), (Q4K, 600, 1024)])
@pytest.mark.parametrize("acc", [False, True])
def test_typed_fast_gemv_matches_fp32(backend, t, dt, N, K, acc):
    """Batch-1 fast GEMV with x and c of one 16-bit type, read and written directly by the K-across-lanes kernel
    (600x1024 q4_k, 4 blocks a row, runs on another kernel through fp32 copies): the bits of
    round(c_widened (+) the fp32 fast GEMV of the widened x), and within one 16-bit step (plus the fast-mode bound)
    of the rounded exact product."""
    raw = synth.quant_weights(dt, N, K, seed=N + 7 * K, outliers=0.01 if dt in (Q4K, Q6K) else 0.0)
    w = backend.FromQuantized(dt, raw, N, K)
    rng = np.random.default_rng(N + K)
    xa, xw = _in(t, rng.standard_normal(K).astype(np.float32))
    ca, cw = _in(t, (rng.standard_normal(N) * 5).astype(np.float32))
    got = _run(backend, w, 1, N, K, xa, t, ca, t, acc, MODE_FAST)
    _same(got, O.round16(t, _fast32(backend, w, N, K, xw, cw, acc)), t)
    exact = O.quant_gemm(dt, 1, N, K, xw.reshape(1, K), raw, cw if acc else None).reshape(-1)
    err = np.max(np.abs(_widen(t, got).astype(np.float64) - O.widen16(t, O.round16(t, exact))) / (1.0 + np.abs(exact)))
    assert err <= (1e-2 if t == BF16 else 2e-3), err
    w.release()


@pytest.mark.parametrize("t", [F16, BF16])
@pytest.mark.parametrize("scale", [1e-6, 2e-5, 3e3, 1e4])
@pytest.mark.parametrize("mode", [MODE_FAST, MODE_EXACT])
def test_typed_rounding_ranges(backend, t, scale, mode):
    """Outputs across the f16 subnormal range (scale 1e-6, 2e-5) and around its overflow edge (3e3, 1e4: row sums
    past 65504 round to Inf): the bits of the oracle's rounding of the fp32 call on the widened activations, for the
    fused batch-1 GEMV and the staged path (exact mode), both with c accumulated."""
    N, K = 4096, 4096
    raw = synth.quant_weights(Q4K, N, K, seed=31, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N, K)
    rng = np.random.default_rng(int(scale * 1e6) % 1000 + 5)
    xa, xw = _in(t, (rng.standard_normal(K) * scale).astype(np.float32))
    ca, cw = _in(t, (rng.standard_normal(N) * scale).astype(np.float32))
    got = _run(backend, w, 1, N, K, xa, t, ca, t, True, mode)
    if mode == MODE_FAST:
        y = _fast32(backend, w, N, K, xw, cw, True)
    else:
        y = O.quant_gemm(Q4K, 1, N, K, xw.reshape(1, K), raw, cw).reshape(-1)
    want = O.round16(t, y)
    _same(got, want, t)
    if t == F16 and scale < 1e-4:
        assert np.sum(np.abs(O.widen16(F16, want)) < 6.1e-5) > 100  # the subnormal range is exercised
    if t == F16 and scale > 1e3:
        assert np.isinf(O.widen16(F16, want)).any() or scale < 5e3
    w.release()


@pytest.mark.parametrize("t", [F16, BF16])
def test_typed_special_values(backend, t):
    """NaN / Inf activations give the NaN / Inf outputs of the fp32 call through the rounding (the oracle's product
    in exact mode, the fp32 fast GEMV of the widened activations in fast mode); f16
    outputs beyond 65504 round to Inf; a call of zero rows leaves c alone."""
    N, K = 96, 1024
    raw = synth.quant_weights(Q4K, N, K, seed=5, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N, K)
    rng = np.random.default_rng(9)
    x = rng.standard_normal(K).astype(np.float32)
    for mode in (MODE_EXACT, MODE_FAST):
        for bad in (np.nan, np.inf, -np.inf):
            xb = x.copy()
            xb[17] = bad
            xa, xw = _in(t, xb)
            got = _widen(t, _run(backend, w, 1, N, K, xa, t, np.zeros(N, np.uint16), t, False, mode))
            if mode == MODE_EXACT:
                want = O.quant_gemm(Q4K, 1, N, K, xw.reshape(1, K), raw).reshape(-1)
            else:
                want = _fast32(backend, w, N, K, xw, np.zeros(N, np.float32), False)
            assert np.array_equal(np.isnan(got), np.isnan(want))
            assert np.array_equal(np.isinf(got), np.isinf(want))
            assert np.array_equal(np.sign(got[np.isinf(got)]), np.sign(want[np.isinf(want)]))
    if t == F16:  # fp32 activations whose row sums pass the f16 range
        big = x * np.float32(3e5)
        got = _run(backend, w, 1, N, K, big, F32, np.zeros(N, np.uint16), F16, False, MODE_EXACT)
        want = O.round16(F16, O.quant_gemm(Q4K, 1, N, K, big.reshape(1, K), raw).reshape(-1))
        assert np.isinf(O.widen16(F16, want)).any() and np.isfinite(O.widen16(F16, want)).any()
        _same(got, want, F16)
    c0 = O.round16(t, np.array([1.5, -0.0, 3.0], np.float32))
    cb = backend.ctx.to_device(c0)
    backend.GemmTyped(0, 3, K, cb, t, w, cb, t, accumulate=False)
    _same(cb.download(np.uint16, 3), c0, t)
    cb.free()
    w.release()


def test_typed_unaligned_and_refusals(backend):
    """A 16-bit x that is only 2-byte aligned takes the staged path with the same bits; bad element types are refused
    with TRHIP_ERR_INVALID."""
    from tcb_amd import TrhipError
    N, K = 200, 4096
    raw = synth.quant_weights(Q4K, N, K, seed=21, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N, K)
    rng = np.random.default_rng(2)
    xa, xw = _in(BF16, rng.standard_normal(K).astype(np.float32))
    xb = backend.ctx.alloc(K * 2 + 16)
    xb.upload(xa, byte_offset=2)
    cb = backend.ctx.alloc(N * 2)
    backend.GemmTyped(1, N, K, (xb, 2), BF16, w, cb, BF16, mode=MODE_FAST)
    got = cb.download(np.uint16, N)
    aligned = _run(backend, w, 1, N, K, xa, BF16, np.zeros(N, np.uint16), BF16, False, MODE_FAST)
    _same(got, aligned, BF16)
    with pytest.raises(TrhipError):
        backend.GemmTyped(1, N, K, xb, 7, w, cb, BF16)
    with pytest.raises(TrhipError):
        backend.GemmTyped(1, N, K, xb, BF16, w, cb, -1)
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("t", [F16, BF16])
@pytest.mark.parametrize("M,mode", [(1, MODE_FAST), (1, MODE_EXACT), (6, MODE_FAST)])
def test_typed_row_slice(backend, t, M, mode):
    """A row slice of the store (row0 = 7, N = 2000 of 2100 rows): the bits of the same call on the fp32 entry
    point over the widened activations, rounded once."""
    R, N, K, row0 = 2100, 2000, 4096, 7
    raw = synth.quant_weights(Q4K, R, K, seed=77, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, R, K)
    rng = np.random.default_rng(M + 3)
    xa, xw = _in(t, rng.standard_normal(M * K).astype(np.float32))
    ca, cw = _in(t, rng.standard_normal(M * N).astype(np.float32))
    xb, cb = backend.ctx.to_device(xa), backend.ctx.to_device(ca)
    backend.GemmTyped(M, N, K, xb, t, w, cb, t, row0=row0, accumulate=True, mode=mode)
    got = cb.download(np.uint16, M * N)
    xb.free()
    cb.free()
    xb, cb = backend.ctx.to_device(xw), backend.ctx.to_device(cw)
    backend.Gemm(M, N, K, xb, w, cb, row0=row0, mode=mode)
    want = O.round16(t, cb.download(np.float32, M * N))
    xb.free()
    cb.free()
    _same(got, want, t)
    w.release()


def _fast32m(backend, w, M, N, K, xw, cw, acc, row0=0):
    """The fp32 fast call of M rows on the widened activations (on the widened c when accumulating)."""
    xb, cb = backend.ctx.to_device(xw), backend.ctx.to_device(cw)
    (backend.Gemm if acc else backend.GemmSet)(M, N, K, xb, w, cb, row0=row0, mode=MODE_FAST)
    y = cb.download(np.float32, M * N)
    xb.free()
    cb.free()
    return y


@pytest.mark.parametrize("t", [F16, BF16])
@pytest.mark.parametrize("dt,M,N,K", [(Q4K, 16, 14336, 4096), (Q4K, 5, 1000, 4096), (Q4K, 9, 4096, 14336),
                                      (Q4, 2, 4096, 4096), (Q4, 8, 300, 2048), (Q4K, 16, 28672, 1024)])
@pytest.mark.parametrize("acc", [False, True])
def test_typed_batched_fast_bits(backend, t, dt, M, N, K, acc):
    """Batched decode (q4_k 5..16 rows, q4_0 2..16) with x and c of one 16-bit type, read and written by the batched
    kernels themselves (one K slice, several slices summed by the last workgroup, 128-row tiles): the bits of the
    fp32 fast call on the widened activations and c, rounded once."""
    raw = synth.quant_weights(dt, N, K, seed=N + M, outliers=0.01 if dt == Q4K else 0.0)
    w = backend.FromQuantized(dt, raw, N, K)
    rng = np.random.default_rng(M * 3 + N)
    xa, xw = _in(t, rng.standard_normal(M * K).astype(np.float32))
    ca, cw = _in(t, (rng.standard_normal(M * N) * 3).astype(np.float32))
    got = _run(backend, w, M, N, K, xa, t, ca, t, acc, MODE_FAST)
    _same(got, O.round16(t, _fast32m(backend, w, M, N, K, xw, cw, acc)), t)
    w.release()


@pytest.mark.parametrize("t", [F16, BF16])
def test_typed_batched_nan_rows_and_alignment(backend, t):
    """NaN / Inf activation rows (the exact float fallback reads the 16-bit x), a row slice, and an x that is only
    2-byte aligned (copied first): the bits of the fp32 fast call on the widened values, rounded once."""
    R, N, K, M, row0 = 1200, 1000, 4096, 7, 100
    raw = synth.quant_weights(Q4K, R, K, seed=5, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, R, K)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[2, 100] = np.nan
    x[5, 4000] = np.inf
    xa, xw = _in(t, x.reshape(-1))
    ca, cw = _in(t, rng.standard_normal(M * N).astype(np.float32))
    xb = backend.ctx.alloc(M * K * 2 + 16)
    xb.upload(xa, byte_offset=2)
    cb = backend.ctx.to_device(ca)
    backend.GemmTyped(M, N, K, (xb, 2), t, w, cb, t, row0=row0, accumulate=True, mode=MODE_FAST)
    got = cb.download(np.uint16, M * N)
    xb.free()
    cb.free()
    _same(got, O.round16(t, _fast32m(backend, w, M, N, K, xw, cw, True, row0=row0)), t)
    w.release()
