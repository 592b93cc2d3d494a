"""The allocation-free act-quant entry point (trhip_gemm_q_actq_noalloc, static device scratch) through the C-ABI:
the same bits as trhip_gemm_q_actq on calls in a row, each smaller than the one before (so the scratch holds the last
call's contents; one q4_k call takes the tiled 128-row prefill kernel), in set and accumulate mode, with an unaligned
activation pointer and a NaN row, and sizes beyond the scratch refused before anything runs."""
import numpy as np
import pytest

import oracle as O
from conftest import same_bits
from tcb_amd import Q4, Q4K, Q6K, _lib, synth

pytestmark = pytest.mark.gpu

CASES = {Q4K: [(512, 4096, 4096), (256, 24576, 1024), (40, 300, 2048)], Q4: [(96, 1024, 4096), (9, 130, 1024)],
         Q6K: [(64, 1024, 4096), (5, 77, 2048)]}


@pytest.mark.parametrize("dt", [Q4K, Q4, Q6K])
def test_noalloc_matches_actq(backend, dt):
    L = _lib.lib()
    h = backend.ctx.h
    for i, (M, N, K) in enumerate(CASES[dt]):
        print("noalloc case dt=%d M=%d N=%d K=%d" % (dt, M, N, K), flush=True)
        raw = synth.quant_weights(dt, N, K, seed=90 + i, outliers=0.01 if dt != Q4 else 0.0)
        w = backend.FromQuantized(dt, raw, N, K)
        X = synth.activations(M, K, seed=91 + i)
        X[M // 2, 7] = np.nan
        off = 4 * i  # the second call takes an x that is not 16-byte aligned (copied inside the scratch)
        xb = backend.ctx.alloc(M * K * 4 + 16)
        xb.upload(X, byte_offset=off)
        c0 = synth.activations(M, N, seed=92 + i).reshape(-1)
        for acc in (0, 1):
            ca, cb = backend.ctx.to_device(c0), backend.ctx.to_device(c0)
            assert L.trhip_gemm_q_actq_noalloc(h, w.h, 0, N, xb.addr(off), cb.addr(), M, K, acc) == 0, \
                L.trhip_last_error(h)
            assert L.trhip_gemm_q_actq(h, w.h, 0, N, xb.addr(off), ca.addr(), M, K, acc) == 0
            got = cb.download(np.float32, M * N)
            same_bits(got, ca.download(np.float32, M * N))
            if M * N * K <= 2e8:
                same_bits(got, O.quant_gemm_act(dt, M, N, K, X, raw, c0 if acc else None))
            for b in (ca, cb):
                b.free()
        xb.free()
        w.release()


def test_noalloc_refuses_beyond_scratch(backend):
    L = _lib.lib()
    h = backend.ctx.h
    M, N, K = 4096, 8, 14336  # about 75 MB of scratch
    w = backend.FromQuantized(Q4K, synth.quant_weights(Q4K, N, K, seed=1, outliers=0.01), N, K)
    xb, cb = backend.ctx.alloc(M * K * 4), backend.ctx.alloc(M * N * 4)
    assert L.trhip_gemm_q_actq_noalloc(h, w.h, 0, N, xb.addr(), cb.addr(), M, K, 0) == 1
    assert b"scratch" in L.trhip_last_error(h)
    for b in (xb, cb):
        b.free()
    w.release()
