"""CPU tests of the boundary and host logic: the C-ABI library loads and exports every entry point that
include/trhip.h declares, the Python binding covers the same set, error paths fail loudly, and the synthetic
encoders used by the benchmark produce well-formed blocks. No compute call is made (there is no GPU here)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trhip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(trhip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("trhip_init", "trhip_wstore_create", "trhip_gemm_q", "trhip_gemm_q_actq", "trhip_gemm_q_actq_mode",
                 "trhip_open_q",
                 "trhip_embedding_q", "trhip_check_quant_scales", "trhip_strerror", "trhip_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from tcb_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    from tcb_amd import _lib
    assert sorted(n for n, _, _ in _lib.SIGNATURES) == declared()


def test_error_strings_and_version():
    from tcb_amd import _lib
    lib = _lib.lib()
    assert lib.trhip_version() > 0
    for code in range(0, 8):
        s = lib.trhip_strerror(code)
        assert s and len(s) >= 2
    assert b"unknown" in lib.trhip_strerror(999).lower()


def test_check_quant_scales_abi_matches_oracle():
    """trhip_check_quant_scales runs on the host (load gate, quant.go:108-128): same answer as the oracle."""
    from tcb_amd import _lib
    lib = _lib.lib()
    for dt in (1, 2, 3, 4):
        size = O.BLOCK[dt][1]
        for at in {1: [0], 2: [0], 3: [0, 2], 4: [208]}[dt]:
            raw = np.zeros(4 * size, np.uint8)
            raw[2 * size + at], raw[2 * size + at + 1] = 0x00, 0x7C
            bad = ctypes.c_int64(0)
            assert lib.trhip_check_quant_scales(dt, raw.ctypes.data_as(ctypes.c_void_p), raw.size, ctypes.byref(bad)) == 0
            assert bad.value == 2 == O.check_quant_scales(dt, raw)
    bad = ctypes.c_int64(0)
    assert lib.trhip_check_quant_scales(9, None, 0, ctypes.byref(bad)) != 0


@pytest.mark.parametrize("dt", [1, 2, 3, 4])
def test_check_quant_scales_large_inputs(dt):
    """Inputs of 4 MB and more are scanned in eight contiguous ranges by eight threads: the answer is still the
    first bad block (the oracle's single pass), with bad blocks in one range, in several, at the range edges, in the
    last block, and none. A short tail block (not a whole block: the reference's slice of it would panic,
    quant.go:108-128) has its scale checked only where the scale's bytes lie inside the input."""
    from tcb_amd import _lib
    lib = _lib.lib()
    size = O.BLOCK[dt][1]
    at = {1: 0, 2: 0, 3: 2, 4: 208}[dt]
    nblk = (5 << 20) // size + 3
    part = (nblk + 7) // 8
    cases = [[], [nblk - 1], [7 * part], [7 * part - 1, 7 * part], [3 * part + 5, 6 * part, part - 1], [0, nblk - 1],
             [2 * part + 1, 5 * part + 2]]
    for bads in cases:
        raw = np.zeros(nblk * size, np.uint8)
        for b in bads:
            raw[b * size + at], raw[b * size + at + 1] = 0x00, 0xFC  # -Inf
        for nbytes in (raw.size, raw.size - size // 2):  # whole blocks, then a short tail block
            bad = ctypes.c_int64(0)
            assert lib.trhip_check_quant_scales(dt, raw.ctypes.data_as(ctypes.c_void_p), nbytes, ctypes.byref(bad)) == 0
            if nbytes == raw.size:
                assert bad.value == O.check_quant_scales(dt, raw) == (min(bads) if bads else -1), (dt, bads)
            else:  # the tail's scale counts only if its two bytes are inside the input
                seen = [x for x in bads if x * size + at + 2 <= nbytes]
                assert bad.value == (min(seen) if seen else -1), (dt, bads, nbytes)


def test_check_quant_scales_concurrent_and_forked():
    """The host scan's worker pool serves one split at a time: scans from several threads at once all give the
    first bad block, and a forked child (which has none of the pool's workers) scans on its own thread."""
    import threading
    from tcb_amd import _lib
    lib = _lib.lib()
    dt, size = 3, O.BLOCK[3][1]
    nblk = (6 << 20) // size
    raws, want = [], []
    for i in range(6):
        raw = np.zeros(nblk * size, np.uint8)
        b = (i * 977 + 11) % nblk
        raw[b * size + 2], raw[b * size + 3] = 0x00, 0x7E  # NaN dmin
        raws.append(raw)
        want.append(b)
    got = [None] * len(raws)

    def scan(i):
        for _ in range(5):
            bad = ctypes.c_int64(0)
            assert lib.trhip_check_quant_scales(dt, raws[i].ctypes.data_as(ctypes.c_void_p), raws[i].size,
                                                ctypes.byref(bad)) == 0
            got[i] = bad.value

    ts = [threading.Thread(target=scan, args=(i,)) for i in range(len(raws))]
    for t in ts:
        t.start()
    for t in ts:
        t.join(60)
    assert got == want
    r, w = os.pipe()
    pid = os.fork()
    if pid == 0:  # child: scan, report, exit without running the parent's cleanup
        bad = ctypes.c_int64(0)
        lib.trhip_check_quant_scales(dt, raws[1].ctypes.data_as(ctypes.c_void_p), raws[1].size, ctypes.byref(bad))
        os.write(w, str(bad.value).encode())
        os._exit(0)
    os.close(w)
    import select
    ready, _, _ = select.select([r], [], [], 60)
    assert ready, "the forked child's scan did not finish"
    assert int(os.read(r, 64)) == want[1]
    os.waitpid(pid, 0)


def test_missing_library_fails_loudly(tmp_path):
    from tcb_amd import _lib
    with pytest.raises(ImportError):
        _lib.load(str(tmp_path / "libtrhip.so"))


def test_null_context_is_refused():
    from tcb_amd import _lib
    lib = _lib.lib()
    assert lib.trhip_gemm_q(None, None, 0, 1, None, None, 1, 32, 1, 0) != 0
    assert lib.trhip_gemm_q_actq(None, None, 0, 1, None, None, 1, 256, 1) != 0
    assert lib.trhip_gemm_q_actq_mode(None, None, 0, 1, None, None, 1, 256, 1, 1) != 0
    assert lib.trhip_sync(None) != 0


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one" in r.stderr.lower()


# ---------------------------------------------------------------- synthetic encoders (benchmark inputs)
def test_q4_0_encoder_zero_block():
    """llama.cpp quantize_row_q4_0_ref on a zero block: d = -0/8 = -0 (fp16 0x8000), codes 8 (0x88)."""
    from tcb_amd import synth
    raw = synth.encode_q4_0(np.zeros((1, 32), np.float32))
    assert list(raw[:2]) == [0x00, 0x80]
    assert np.all(raw[2:] == 0x88)
    assert np.all(O.dequant(2, raw) == 0)


def test_q8_0_encoder_known_block():
    """d = amax/127 (fp16), code = round-half-away(x/d)."""
    from tcb_amd import synth
    x = np.zeros((1, 32), np.float32)
    x[0, 0], x[0, 1], x[0, 2] = 127.0, -63.5, 0.5
    raw = synth.encode_q8_0(x)
    assert list(raw[:2]) == [0x00, 0x3C]  # d = 1.0
    assert raw[2:5].view(np.int8).tolist() == [127, -64, 1]


@pytest.mark.parametrize("dt,bound", [(1, 0.008), (2, 0.1), (3, 0.1), (4, 0.025)])
def test_encoders_round_trip(dt, bound):
    """Encoded then dequantized (golden-pinned dequant) stays within the format's error: relative RMS bound."""
    from tcb_amd import synth
    N, K = 8, 1024
    x = synth.weights_f32(N, K, seed=5)  # Gaussian; 1% x10 outliers would widen every bound
    raw = {1: synth.encode_q8_0, 2: synth.encode_q4_0, 3: synth.encode_q4_k, 4: synth.encode_q6_k}[dt](x)
    assert raw.size == N * K // O.BLOCK[dt][0] * O.BLOCK[dt][1]
    assert O.check_quant_scales(dt, raw) == -1
    y = O.dequant(dt, raw).reshape(N, K)
    err = np.sqrt(np.mean((y.astype(np.float64) - x) ** 2)) / np.sqrt(np.mean(x.astype(np.float64) ** 2))
    assert err < bound, err
