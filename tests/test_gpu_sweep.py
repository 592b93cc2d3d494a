"""GPU parity for the full single-token decode sweep of a Llama-3-8B-shaped model: the q6_k output head
128256 x 4096 at batch 1 and 16, and the per-layer linears captured into one HIP graph and replayed.

The layer wiring follows lib/pretrained.tr:279-310 (q, k, v, o, gate, up, down per layer, then the output head);
the merged variant uses the reference's merged projections (lib/layers.tr:240-262: [q | k | v], [gate | up] with
the SwiGLU gate). Exact mode is held bit for bit to the oracle (quantDot / quantGemmPanels order); fast mode to
1e-4 by the reference's |a - b| / (1 + |b|) (gpu/helpers_test.go:82), as gpu/behavior_quant_test.go:283-304 holds
its GEMV against the opened weights. Every replay of a graph must equal the eager run bit for bit.
"""
import ctypes
import functools

import numpy as np
import pytest

import oracle as O
from conftest import rel_err, same_bits
from tcb_amd import BLOCK, MODE_EXACT, MODE_FAST, Q4K, Q6K, QuantBackend, QuantWeight, _lib, synth

pytestmark = pytest.mark.gpu

TOL = 1e-4  # fast-mode bound for the K-quants
LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
VOCAB, HIDDEN = 128256, 4096
LAYERS = 2


@functools.lru_cache(maxsize=None)
def _base(dt, K):
    """2048 encoded rows of N(0, 0.02) weights with 1% outliers x10."""
    return synth.quant_weights(dt, 2048, K, seed=500 + 10 * dt + K, outliers=0.01).reshape(2048, -1)


def rows_of(dt, N, K, seed):
    """N rows of encoded blocks: base rows in a seeded order, each block's fp16 scale d with its three lowest mantissa
    bits xor-ed by a per-row pattern (d changes by under 0.7%), so rows and stores do not share bytes."""
    base = _base(dt, K)
    pick = np.random.default_rng(seed).integers(0, base.shape[0], N)
    out = base[pick]
    blk = out.reshape(N, K // BLOCK[dt][0], BLOCK[dt][1])
    d_lo = 0 if dt == Q4K else 208  # low byte of the fp16 d
    pat = ((np.arange(N, dtype=np.uint64) * 2654435761 + seed) >> np.uint64(7)) & np.uint64(7)
    blk[:, :, d_lo] ^= pat.astype(np.uint8)[:, None]
    return np.ascontiguousarray(out).reshape(-1)


def activations(batch):
    return {HIDDEN: synth.activations(batch, HIDDEN, seed=7), 14336: synth.activations(batch, 14336, seed=8)}


@pytest.fixture(scope="module")
def head(backend):
    raw = rows_of(Q6K, VOCAB, HIDDEN, seed=77)
    w = backend.FromQuantized(Q6K, raw, VOCAB, HIDDEN)
    yield raw, w
    w.release()


@pytest.fixture(scope="module")
def layers(backend):
    out = []
    for li in range(LAYERS):
        ws = []
        for si, (name, n, k) in enumerate(LAYER):
            raw = rows_of(Q4K, n, k, seed=1000 * li + si)
            ws.append((raw, backend.FromQuantized(Q4K, raw, n, k)))
        out.append(ws)
    yield out
    for ws in out:
        for _, w in ws:
            w.release()


@pytest.fixture(scope="module")
def want():
    """Oracle results, computed once per key."""
    cache = {}

    def get(key, fn):
        if key not in cache:
            cache[key] = fn()
        return cache[key]

    return get


@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("mode", [MODE_EXACT, MODE_FAST])
def test_head_q6k_128256(backend, head, want, M, mode):
    """The q6_k output head 128256 x 4096 on encoded weights, every row: exact bit-identical, fast within 1e-4."""
    raw, w = head
    X = activations(M)[HIDDEN]
    ref = want(("head", M), lambda: O.quant_gemm(Q6K, M, VOCAB, HIDDEN, X, raw))
    xb, cb = backend.ctx.to_device(X), backend.ctx.alloc(M * VOCAB * 4)
    backend.GemmSet(M, VOCAB, HIDDEN, xb, w, cb, mode=mode)
    got = cb.download(np.float32, M * VOCAB)
    if mode == MODE_EXACT:
        same_bits(got, ref)
    else:
        assert rel_err(got, ref) <= TOL
    for b in (xb, cb):
        b.free()


def _capture(backend, fn):
    L = _lib.lib()
    assert L.trhip_graph_begin(backend.ctx.h) == 0
    try:
        fn()
    finally:
        g = ctypes.c_void_p()
        rc = L.trhip_graph_end(backend.ctx.h, ctypes.byref(g))
    assert rc == 0, L.trhip_last_error(backend.ctx.h)
    return g


def _replays_equal_eager(backend, g, bufs, eager, between):
    """Replay the graph three times, with the outputs cleared to NaN bytes and other eager work between replays;
    every replay must give the eager bits."""
    L = _lib.lib()
    for r in range(3):
        for b in bufs:
            b.fill(0xFF)
        between(r)
        assert L.trhip_graph_launch(backend.ctx.h, g) == 0
        backend.ctx.sync()
        for b, e in zip(bufs, eager):
            same_bits(b.download(np.float32, e.size), e)


@pytest.mark.parametrize("batch", [1, 16])
@pytest.mark.parametrize("mode", [MODE_EXACT, MODE_FAST])
@pytest.mark.parametrize("merged", [False, True])
def test_decode_sweep_graph(backend, layers, head, want, batch, mode, merged):
    """Two layers of all seven Llama-3-8B linears (distinct q4_k weights) and the q6_k head, back to back on one
    stream and captured into one graph (the decode sweep's launch sequence, sharing the context's workspaces).
    Replays equal the eager run bit for bit; every GEMV is bit-identical (exact) or within 1e-4 (fast) of the
    oracle. Merged: [q | k | v] and [gate | up] stores, the gate/up product followed by the SwiGLU gate."""
    xh = activations(batch)
    xs = {k: backend.ctx.to_device(v) for k, v in xh.items()}
    hraw, hw = head

    def ref(li, si):
        _, n, k = LAYER[si]
        return want((li, si, batch), lambda: O.quant_gemm(Q4K, batch, n, k, xh[k], layers[li][si][0]))

    href = want(("head", batch), lambda: O.quant_gemm(Q6K, batch, VOCAB, HIDDEN, xh[HIDDEN], hraw))
    by = {name: i for i, (name, _, _) in enumerate(LAYER)}
    extra = []
    if not merged:
        outs = [[backend.ctx.alloc(batch * n * 4) for _, n, _ in LAYER] for _ in range(LAYERS)]

        def step():
            for li in range(LAYERS):
                for si, (_, n, k) in enumerate(LAYER):
                    backend.GemmSet(batch, n, k, xs[k], layers[li][si][1], outs[li][si], mode=mode)
            backend.GemmSet(batch, VOCAB, HIDDEN, xs[HIDDEN], hw, hout, mode=mode)
    else:
        stores = []
        for li in range(LAYERS):
            ws = [w for _, w in layers[li]]
            qkv = QuantWeight.Concat([ws[by["q"]], ws[by["k"]], ws[by["v"]]])
            gu = QuantWeight.Concat([ws[by["gate"]], ws[by["up"]]])
            stores.append((qkv, ws[by["o"]], gu, ws[by["down"]]))
        extra = [s for st in stores for s in (st[0], st[2])]
        outs = [[backend.ctx.alloc(batch * n * 4) for n in (6144, 4096, 14336, 4096)] for _ in range(LAYERS)]

        def step():
            for li, (qkv, o, gu, down) in enumerate(stores):
                backend.GemmSet(batch, 6144, HIDDEN, xs[HIDDEN], qkv, outs[li][0], mode=mode)
                backend.GemmSet(batch, 4096, HIDDEN, xs[HIDDEN], o, outs[li][1], mode=mode)
                backend.GemmSwiGLU(batch, HIDDEN, xs[HIDDEN], gu, outs[li][2], mode=mode)
                backend.GemmSet(batch, 4096, 14336, xs[14336], down, outs[li][3], mode=mode)
            backend.GemmSet(batch, VOCAB, HIDDEN, xs[HIDDEN], hw, hout, mode=mode)

    hout = backend.ctx.alloc(batch * VOCAB * 4)
    bufs = [b for row in outs for b in row] + [hout]
    step()
    backend.ctx.sync()
    eager = [b.download(np.float32, b.nbytes // 4) for b in bufs]
    g = _capture(backend, step)
    side_x = backend.ctx.to_device(synth.activations(3, HIDDEN, seed=99))
    side_c = backend.ctx.alloc(3 * 4096 * 4)

    def between(r):  # eager work of the program itself between replays
        backend.GemmSet(3, 4096, HIDDEN, side_x, layers[r % LAYERS][by["o"]][1], side_c, mode=mode)
        backend.ctx.sync()

    try:
        _replays_equal_eager(backend, g, bufs, eager, between)
    finally:
        _lib.lib().trhip_graph_destroy(g)

    def check(got, ref_):
        if mode == MODE_EXACT:
            same_bits(got, ref_)
        else:
            assert rel_err(got, ref_) <= TOL

    if not merged:
        for li in range(LAYERS):
            for si in range(len(LAYER)):
                check(eager[li * len(LAYER) + si], ref(li, si))
    else:
        for li, (qkv, o, gu, down) in enumerate(stores):
            e = eager[4 * li:4 * li + 4]
            check(e[0], np.concatenate([ref(li, by["q"]), ref(li, by["k"]), ref(li, by["v"])], axis=1))
            check(e[1], ref(li, by["o"]))
            check(e[3], ref(li, by["down"]))
            gu_ref = np.concatenate([ref(li, by["gate"]), ref(li, by["up"])], axis=1)
            if mode == MODE_EXACT:
                same_bits(e[2], O.swiglu(gu_ref, batch, 14336))
            else:  # the gated output is the gate applied to the unfused fast product of the merged store, bit for bit
                gb = backend.ctx.alloc(batch * 28672 * 4)
                backend.GemmSet(batch, 28672, HIDDEN, xs[HIDDEN], gu, gb, mode=mode)
                gu_fast = gb.download(np.float32, batch * 28672)
                gb.free()
                assert rel_err(gu_fast, gu_ref) <= TOL
                same_bits(e[2], O.swiglu(gu_fast, batch, 14336))
    check(eager[-1], href)
    for b in bufs + list(xs.values()) + [side_x, side_c]:
        b.free()
    for w in extra:
        w.release()


def test_graph_replay_after_workspace_growth():
    """A graph captured while the context's workspaces are small keeps working after an eager call grows them
    (the retired buffers live until the last graph is gone), also when new allocations follow and are filled. Calls
    that wait for the stream are refused during capture, and a graph replays only on its own context."""
    L = _lib.lib()
    tb = QuantBackend(0)  # a fresh context: empty workspaces
    other = QuantBackend(0)
    try:
        raw = synth.quant_weights(Q4K, 1024, 4096, seed=3, outliers=0.01)
        w = tb.FromQuantized(Q4K, raw, 1024, 4096)
        gu = tb.FromQuantized(Q4K, synth.quant_weights(Q4K, 2048, 4096, seed=4, outliers=0.01), 2048, 4096)
        X = synth.activations(16, 4096, seed=5)
        xb, cb, sb = tb.ctx.to_device(X), tb.ctx.alloc(16 * 1024 * 4), tb.ctx.alloc(16 * 1024 * 4)

        def step():  # fast M = 16 (digits + slice partials in the workspace), merged SwiGLU (the second workspace)
            tb.GemmSet(16, 1024, 4096, xb, w, cb, mode=MODE_FAST)
            tb.GemmSwiGLU(16, 4096, xb, gu, sb, mode=MODE_FAST)

        step()
        tb.ctx.sync()
        eager = [cb.download(np.float32, 16 * 1024), sb.download(np.float32, 16 * 1024)]
        assert L.trhip_graph_begin(tb.ctx.h) == 0
        step()
        assert L.trhip_sync(tb.ctx.h) == 1  # refused while capturing
        host = np.zeros(4, np.float32)
        assert L.trhip_d2h(tb.ctx.h, host.ctypes.data_as(ctypes.c_void_p), cb.addr(), 16) == 1
        g = ctypes.c_void_p()
        assert L.trhip_graph_end(tb.ctx.h, ctypes.byref(g)) == 0
        # grow both workspaces eagerly, then allocate and fill device memory where freed buffers would be reused
        big = tb.ctx.to_device(synth.activations(2048, 4096, seed=6))
        big_out = tb.ctx.alloc(2048 * 1024 * 4)
        tb.GemmActQuant(2048, 1024, 4096, big, w, big_out, accumulate=False)
        gu_big = tb.ctx.alloc(256 * 1024 * 4)
        tb.GemmSwiGLU(256, 4096, big, gu, gu_big, mode=MODE_FAST)
        tb.ctx.sync()
        junk = [tb.ctx.alloc(8 << 20) for _ in range(8)]
        for j in junk:
            j.fill(0xFF)
        tb.ctx.sync()
        assert L.trhip_graph_launch(other.ctx.h, g) == 1  # another context's graph is refused
        for r in range(3):
            cb.fill(0)
            sb.fill(0)
            assert L.trhip_graph_launch(tb.ctx.h, g) == 0
            tb.ctx.sync()
            same_bits(cb.download(np.float32, 16 * 1024), eager[0])
            same_bits(sb.download(np.float32, 16 * 1024), eager[1])
        assert L.trhip_graph_destroy(g) == 0
        for b in [xb, cb, sb, big, big_out, gu_big] + junk:
            b.free()
        w.release()
        gu.release()
    finally:
        other.close()
        tb.close()
