"""GPU tests of the library's life-cycle rules and host-side upload path, through the C-ABI:

- store creation copies every byte of a pageable source at sizes where the host copy's thread split is ragged,
  and applies the scale gate (tensor/quant.go:108-128, H6686) chunk by chunk beside the upload;
- a context refuses to be destroyed while stores or graphs made on it are alive;
- a kernel's dynamic-LDS cap follows the largest request, whatever order the shapes come in.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle as O
from conftest import same_bits
from tcb_amd import BLOCK, Q4K, Q6K, Q8, TrhipError, _lib
from tcb_amd.backend import Context, QuantWeight

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
UPLOAD_CHUNK = 8 << 20  # bytes per upload chunk of trhip_wstore_create
ERR_INVALID, ERR_BAD_SCALE = 1, 7


def _chunk_blocks(dt):
    return UPLOAD_CHUNK // BLOCK[dt][1] // 8 * 8


def test_store_ragged_pageable_upload(backend):
    """q6_k 1431 x 3840 is 4,507,650 bytes: above the size where the host copy is split over eight threads, and not
    a multiple of eight. Every byte reaches the device: ToRaw returns the source, and OpenQuant of the last row (whose
    last block's fp16 d is the final two bytes) equals the oracle's dequantization."""
    dt, N, K = Q6K, 1431, 3840
    raw = O.random_quant(dt, 11, N * K // 256)
    assert raw.nbytes == 4507650 and raw.nbytes % 8 == 2
    w = QuantWeight(backend.ctx, dt, raw, N, K)
    assert np.array_equal(w.ToRaw(), raw)
    out = backend.ctx.alloc(K * 4)
    backend.OpenQuant(out, w, offset=(N - 1) * K, n=K)
    same_bits(out.download(np.float32, K), O.dequant(dt, raw[-(K // 256) * 210:]))
    out.free()
    w.release()


@pytest.mark.parametrize("pinned", [False, True])
@pytest.mark.parametrize("dt", [Q8, Q4K, Q6K])
def test_store_scale_gate_across_chunks(dt, pinned):
    """A NaN/Inf scale in the last block of the first upload chunk, the first of the second or inside the third is
    refused with H6686 and the index the host gate gives; no store is left behind (the context can then be
    destroyed), and a good store made afterwards on the same context round-trips."""
    elems, size = BLOCK[dt]
    per = _chunk_blocks(dt)
    K = 4096
    nb = K // elems
    N = (3 * per + 17) // nb
    ctx = Context(0)
    try:
        good = O.random_quant(dt, 5, N * nb)
        at = {Q8: 0, Q4K: 2, Q6K: 208}[dt]
        for bad_block in (per - 1, per, 2 * per + 9):
            raw = good.copy()
            raw[bad_block * size + at:bad_block * size + at + 2] = (0x00, 0xFC)  # -Inf
            assert O.check_quant_scales(dt, raw) == bad_block
            if pinned:
                h, p = ctx.host_alloc(raw.nbytes)
                h[:] = raw
                src = h
            with pytest.raises(TrhipError) as e:
                QuantWeight(ctx, dt, src if pinned else raw, N, K)
            if pinned:
                ctx.host_free(p)
            assert e.value.code == ERR_BAD_SCALE
            assert ("block %d " % bad_block) in e.value.detail
        w = QuantWeight(ctx, dt, good, N, K)
        assert np.array_equal(w.ToRaw(N - 3, 3), good[-3 * nb * size:])
        w.release()
    finally:
        assert _lib.lib().trhip_destroy(ctx.h) == 0  # every refused store was dropped
        ctx.h = None


def test_context_outlives_stores_and_graphs():
    """trhip_destroy returns TRHIP_ERR_INVALID while a store or a graph of the context is alive, and the context
    keeps working; it succeeds once they are destroyed."""
    lib = _lib.lib()
    ctx = Context(0)
    N, K = 16, 256
    raw = O.random_quant(Q4K, 3, N * K // 256)
    w = QuantWeight(ctx, Q4K, raw, N, K)
    assert lib.trhip_destroy(ctx.h) == ERR_INVALID
    assert b"still alive" in lib.trhip_last_error(ctx.h)
    assert np.array_equal(w.ToRaw(), raw)
    buf = ctx.alloc(4096)
    assert lib.trhip_graph_begin(ctx.h) == 0
    assert lib.trhip_memset_async(ctx.h, buf.addr(), 0x5A, 4096) == 0
    g = _lib.P()
    assert lib.trhip_graph_end(ctx.h, ctypes.byref(g)) == 0
    w.release()
    assert lib.trhip_destroy(ctx.h) == ERR_INVALID  # the graph is still alive
    assert lib.trhip_graph_launch(ctx.h, g) == 0
    assert np.all(buf.download(np.uint8, 4096) == 0x5A)
    assert lib.trhip_graph_destroy(g) == 0
    buf.free()
    assert lib.trhip_destroy(ctx.h) == 0
    ctx.h = None


_LDS_ORDER_CHILD = r"""
import sys
sys.path[:0] = [%(root)r, %(tests)r]
import numpy as np
import oracle as O
from conftest import rel_err
from tcb_amd import MODE_FAST, Q4K, QuantBackend, synth
b = QuantBackend(0)
N = 1792
for K in (14336, 16384):
    raw = synth.quant_weights(Q4K, N, K, seed=K, outliers=0.01)
    x = synth.activations(1, K, seed=K + 1)
    w = b.FromQuantized(Q4K, raw, N, K)
    xb, cb = b.ctx.to_device(x), b.ctx.alloc(N * 4)
    b.GemmSet(1, N, K, xb, w, cb, mode=MODE_FAST)
    err = rel_err(cb.download(np.float32, N), O.quant_gemm(Q4K, 1, N, K, x, raw).reshape(-1))
    print("K=%%d err=%%.3g" %% (K, err), flush=True)
    assert err <= 1e-4, err
    xb.free(); cb.free(); w.release()
b.close()
print("ok", flush=True)
"""


def test_dyn_lds_cap_follows_largest_request():
    """The fast q4_k GEMV on a 1792-row shard asks for more dynamic LDS at K = 16384 than at K = 14336 on the same
    kernel. Run in that order in a fresh process (the cap is kept per process), both results are within 1e-4 of the
    oracle."""
    code = _LDS_ORDER_CHILD % {"root": ROOT, "tests": os.path.join(ROOT, "tests")}
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
