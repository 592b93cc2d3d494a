"""Fast-mode q4_k (5..16 activation rows) and q4_0 (2..16) products in one launch (rows16.hip): every launch shape
within the tolerance of the oracle, set and accumulate, row slices, ragged N; the K slices summed by the last
workgroup of a row tile give the same bits on every call; the fused SwiGLU gives the bits of the plain call
followed by the gate."""
import numpy as np
import pytest

import oracle as O
from conftest import rel_err, same_bits
from tcb_amd import MODE_EXACT, MODE_FAST, Q4, Q4K, synth
from tcb_amd._lib import KNOB_ROWS16

pytestmark = pytest.mark.gpu
FAST_TOL = {Q4K: 1e-4, Q4: 1e-5}  # the fast-mode bounds: 1e-4 for the K-quants, 1e-5 for q4_0

SHAPES = [(1, 1), (1, 16), (2, 3), (2, 2), (1, 5), (2, 64), (2, 1)]  # (16-row tiles per wave, K slices)


@pytest.mark.parametrize("tpw,S", SHAPES)
@pytest.mark.parametrize("M,N,K,row0", [(16, 1000, 4096, 0), (5, 300, 2048, 7), (9, 77, 3840, 2)])
def test_rows16_shapes(backend, launch_shape, tpw, S, M, N, K, row0):
    raw = synth.quant_weights(Q4K, N + row0, K, seed=N + K + M, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N + row0, K)
    sub = raw.reshape(N + row0, -1)[row0:].reshape(-1)
    launch_shape(KNOB_ROWS16, tpw, S)
    for scale, acc, off in ((1.0, False, 0), (1000.0, True, 4)):
        x = synth.activations(M, K, seed=K + M + 1) * np.float32(scale)
        c0 = synth.activations(M, N, seed=N + 3).reshape(-1)
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
        same_bits(outs[0], outs[1])
        want = O.quant_gemm(Q4K, M, N, K, x, sub, c0 if acc else None).reshape(-1)
        err = rel_err(outs[0] / scale, want / scale)
        assert err <= FAST_TOL[Q4K], (tpw, S, M, N, K, row0, scale, err)
        xb.free()
    w.release()


@pytest.mark.parametrize("tpw,S,M,N,K,row0", [(1, 1, 16, 17000, 1024, 3), (2, 4, 11, 9000, 2048, 0),
                                               (1, 1, 16, 14336, 1024, 0)])
def test_rows16_large_grids(backend, launch_shape, tpw, S, M, N, K, row0):
    """Grids of more workgroups than a 256-CU device has (and one that fits it with one K slice): within the
    tolerance of the oracle."""
    raw = synth.quant_weights(Q4K, N + row0, K, seed=N + M, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N + row0, K)
    sub = raw.reshape(N + row0, -1)[row0:].reshape(-1)
    launch_shape(KNOB_ROWS16, tpw, S)
    x = synth.activations(M, K, seed=K + M + 5)
    xb, cb = backend.ctx.to_device(x), backend.ctx.alloc(M * N * 4)
    backend.GemmSet(M, N, K, xb, w, cb, row0=row0, mode=MODE_FAST)
    want = O.quant_gemm(Q4K, M, N, K, x, sub).reshape(-1)
    assert rel_err(cb.download(np.float32, M * N), want) <= FAST_TOL[Q4K]
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("tpw,S", [(1, 1), (2, 3), (1, 16)])
@pytest.mark.parametrize("M,I,K", [(16, 300, 4096), (7, 129, 1024)])
def test_rows16_swiglu_bits(backend, launch_shape, tpw, S, M, I, K):
    raw = synth.quant_weights(Q4K, 2 * I, K, seed=I + M, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, 2 * I, K)
    X = synth.activations(M, K, seed=K + M)
    launch_shape(KNOB_ROWS16, tpw, S)
    xb, gub, ob = backend.ctx.to_device(X), backend.ctx.alloc(M * 2 * I * 4), backend.ctx.alloc(M * I * 4)
    backend.GemmSet(M, 2 * I, K, xb, w, gub, mode=MODE_FAST)
    gu = gub.download(np.float32, M * 2 * I).reshape(M, 2 * I)
    assert rel_err(gu.reshape(-1), O.quant_gemm(Q4K, M, 2 * I, K, X, raw).reshape(-1)) <= FAST_TOL[Q4K]
    backend.GemmSwiGLU(M, K, xb, w, ob, mode=MODE_FAST)
    same_bits(ob.download(np.float32, M * I), O.swiglu(gu, M, I).reshape(-1))
    for b in (xb, gub, ob):
        b.free()
    w.release()


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_rows16_non_finite_sliced(backend, launch_shape, bad):
    """NaN / Inf rows with K split into slices: each slice's exact float dot, summed in slice order, has the
    exact path's NaN / Inf pattern; the other rows stay within tolerance."""
    M, N, K = 6, 200, 4096
    raw = synth.quant_weights(Q4K, N, K, seed=11, outliers=0.01)
    w = backend.FromQuantized(Q4K, raw, N, K)
    X = synth.activations(M, K, seed=12)
    X[1, 5] = bad
    X[4, 4000] = bad
    X[4, 10] = -bad if not np.isnan(bad) else bad
    launch_shape(KNOB_ROWS16, 1, 4)
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4)
    backend.GemmSet(M, N, K, xb, w, cb, mode=MODE_FAST)
    got = cb.download(np.float32, M * N).reshape(M, N)
    want = O.quant_gemm(Q4K, M, N, K, X, raw).reshape(M, N)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    assert np.array_equal(np.sign(got[~fin & ~np.isnan(want)]), np.sign(want[~fin & ~np.isnan(want)]))
    assert rel_err(got[fin], want[fin]) <= FAST_TOL[Q4K]
    for b in (xb, cb):
        b.free()
    w.release()


@pytest.mark.parametrize("tpw,S", [(1, 1), (1, 16), (2, 3), (1, 5), (2, 64)])
@pytest.mark.parametrize("M,N,K,row0", [(8, 1000, 4096, 0), (5, 300, 2048, 7), (2, 77, 3840, 2), (16, 130, 256, 0)])
def test_rows16_q4_0_shapes(backend, launch_shape, tpw, S, M, N, K, row0):
    """q4_0 at 2..16 rows: one MFMA pair per 32-element block scaled by its d, within the q4_0 bound 1e-5 of the
    oracle on every launch shape, set and accumulate, x1 and x1000, an unaligned x, the same bits on every call."""
    raw = synth.quant_weights(Q4, N + row0, K, seed=N + K + M, outliers=0.01)
    w = backend.FromQuantized(Q4, raw, N + row0, K)
    sub = raw.reshape(N + row0, -1)[row0:].reshape(-1)
    launch_shape(KNOB_ROWS16, tpw, S)
    for scale, acc, off in ((1.0, False, 0), (1000.0, True, 4)):
        x = synth.activations(M, K, seed=K + M + 1) * np.float32(scale)
        c0 = synth.activations(M, N, seed=N + 3).reshape(-1)
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
        same_bits(outs[0], outs[1])
        want = O.quant_gemm(Q4, M, N, K, x, sub, c0 if acc else None).reshape(-1)
        err = rel_err(outs[0] / scale, want / scale)
        assert err <= FAST_TOL[Q4], (tpw, S, M, N, K, row0, scale, err)
        xb.free()
    w.release()


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_rows16_q4_0_non_finite(backend, launch_shape, bad):
    """q4_0 rows holding NaN / Inf (K in slices) take the exact float dot: the exact path's NaN / Inf pattern, the
    other rows within 1e-5; fast differs from exact on some finite output (the matrix-core kernel ran)."""
    M, N, K = 6, 200, 4096
    raw = synth.quant_weights(Q4, N, K, seed=13, outliers=0.01)
    w = backend.FromQuantized(Q4, raw, N, K)
    X = synth.activations(M, K, seed=14)
    X[1, 5] = bad
    X[4, 4000] = bad
    launch_shape(KNOB_ROWS16, 1, 4)
    xb, cb, eb = backend.ctx.to_device(X), backend.ctx.alloc(M * N * 4), backend.ctx.alloc(M * N * 4)
    backend.GemmSet(M, N, K, xb, w, cb, mode=MODE_FAST)
    backend.GemmSet(M, N, K, xb, w, eb, mode=MODE_EXACT)
    got = cb.download(np.float32, M * N).reshape(M, N)
    exact = eb.download(np.float32, M * N).reshape(M, N)
    want = O.quant_gemm(Q4, M, N, K, X, raw).reshape(M, N)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    assert rel_err(got[fin], want[fin]) <= FAST_TOL[Q4]
    assert not np.array_equal(got[fin].view(np.uint32), exact[fin].view(np.uint32))
    for b in (xb, cb, eb):
        b.free()
    w.release()
